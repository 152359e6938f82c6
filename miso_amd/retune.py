"""Engine constants for one MI355X, measured on the attention path.

The reference engine sizes its attention calls with three host constants tuned on an MI50
(gfx906): the decode split cap `AttentionScratch::kMaxSplits = 60`
(src/engine/attention.hpp:44-46, passed to attn_n_splits at src/engine/attention.hip:102), the
prefill chunk `Session::kMaxChunk = 512` (src/engine/model.hpp:58, used by prefill() at
src/engine/model.hip:135) and the prefill threshold `kPrefillMinTokens = 8`
(src/engine/model.hpp:80: fewer tokens are ingested by per-token decode steps,
src/engine/model.hip:168). This module measures what each choice costs on this GPU through the
same entry points the engine calls (miso_amd.attention over the C ABI), without changing any
signature:

  max_splits   one decode call (prep + split + combine) at several contexts, under the engine's
               cap of 60 and under 128 (this build's policy cap: 2 x 128 workgroups fill the
               256 CUs);
  chunk        the attention work of ingesting a P-token prompt (prep_batch + prefill per chunk)
               for several chunk sizes;
  min_tokens   n per-token decode calls (prep + split + combine at lengths L + 1 .. L + n)
               against one prep_batch + prefill of n tokens, at context L;
  prefill_map  the prefill kernel alone (TFLOP/s over the unmasked pairs) for chunk sizes n
               after prefixes pos0: how much of the GPU a chunk of each size fills.

Only the attention kernels are timed: the engine's projections, MoE and DeltaNet layers shift the
real crossover and chunk optimum, so these are the attention path's side of each trade.

    python -m miso_amd.retune [--quick]

prints one JSON object. Inputs are synthetic N(0, 1) data; times are HIP-event times of graph
replays (median of 3), so host launch cost is excluded: the engine launches eagerly, and its
per-call times are at least these.
"""
from __future__ import annotations

import argparse
import json
import math
import sys

H, KV, D = 16, 2, 256
PROJ = 9216  # floats per token of the engine's projection buffer: q+gate 8192 | k 512 | v 512


def _graph(torch, fn, count):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(count):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(count):
            fn(i)
    torch.cuda.synchronize()
    return g


def _time(torch, g, reps):
    """Median over 3 runs of the event time of `reps` replays of g (ms per replay)."""
    g.replay()
    torch.cuda.synchronize()
    runs = []
    for _ in range(3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        runs.append(e0.elapsed_time(e1) / reps)
    return sorted(runs)[1]


class _Weights:
    """Per-layer inputs of attn_prep: norms, RoPE inverse frequencies, one token's projections."""

    def __init__(self, torch, gen, n_tok):
        dev = "cuda"
        self.q_norm = torch.rand(D, generator=gen, device=dev) + 0.5
        self.k_norm = torch.rand(D, generator=gen, device=dev) + 0.5
        self.inv_freq = 1.0 / (1.0e7 ** (torch.arange(32, device=dev, dtype=torch.float32) / 32))
        self.proj = torch.randn(n_tok * PROJ, generator=gen, device=dev)
        self.qg = torch.randn(H * 2 * D, generator=gen, device=dev)
        self.k = torch.randn(KV * D, generator=gen, device=dev)
        self.v = torch.randn(KV * D, generator=gen, device=dev)


def decode_call(A, w, q, core, k, v, sc, length, max_ctx, max_splits):
    """One engine decode step's attention: append the token at position length - 1, then split +
    combine over `length` positions (the engine's attention_decode between its GEMVs)."""
    A.attn_prep(w.qg, w.k, w.v, w.q_norm, w.k_norm, w.inv_freq, k, v, q, length - 1, max_ctx,
                1e-6)
    A.attn_decode(q, w.qg, k, v, core, sc, length, max_ctx, A.attn_n_splits(length, max_splits))


def prefill_call(A, w, q, core, k, v, pos0, n, max_ctx):
    """The engine's attention_prefill between its GEMMs: prep_batch of n tokens, then prefill."""
    A.attn_prep_batch(w.proj[:n * PROJ], w.proj[8192:n * PROJ], w.proj[8704:n * PROJ], w.q_norm,
                      w.k_norm, w.inv_freq, k, v, q, pos0, max_ctx, 1e-6, n, PROJ)
    A.attn_prefill(q, w.proj[:n * PROJ], k, v, core, pos0, n, max_ctx, qg_stride=PROJ)


def sweep_max_splits(torch, A, contexts, caps=(60, 128)):
    out = []
    gen = torch.Generator(device="cuda")
    for L in contexts:
        gen.manual_seed(L)
        w = _Weights(torch, gen, 1)
        cache_bytes = 2 * KV * L * D * 2
        rot = max(1, min(8, math.ceil((384 << 20) / cache_bytes)))  # stream from HBM at long L
        caches = [(torch.randn(KV * L * D, generator=gen, device="cuda").half(),
                   torch.randn(KV * L * D, generator=gen, device="cuda").half())
                  for _ in range(rot)]
        q = torch.empty(H * D, device="cuda")
        core = torch.empty(H * D, device="cuda")
        row = {"ctx": L, "kv_caches_rotated": rot}
        for cap in caps:
            sc = A.DecodeScratch(cap)

            def call(i, cap=cap, sc=sc):
                k, v = caches[i % rot]
                decode_call(A, w, q, core, k, v, sc, L, L, cap)

            g = _graph(torch, call, rot)
            t = _time(torch, g, max(1, 24 // rot)) / rot
            row[f"cap{cap}"] = {"n_splits": A.attn_n_splits(L, cap), "us": round(t * 1e3, 2)}
        row["speedup_128_vs_60"] = round(row["cap60"]["us"] / row["cap128"]["us"], 3)
        out.append(row)
        print(f"[retune] decode ctx {L}: cap 60 {row['cap60']['us']} us, "
              f"cap 128 {row['cap128']['us']} us", file=sys.stderr, flush=True)
        del caches
    return out


def sweep_chunk(torch, A, prompt, chunks):
    out = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(prompt)
    w = _Weights(torch, gen, max(chunks))
    k = torch.zeros(KV * prompt * D, device="cuda").half()
    v = torch.zeros(KV * prompt * D, device="cuda").half()
    q = torch.empty(max(chunks) * H * D, device="cuda")
    core = torch.empty(max(chunks) * H * D, device="cuda")
    for c in chunks:
        calls = prompt // c

        def ingest(_i, c=c, calls=calls):
            for j in range(calls):
                prefill_call(A, w, q, core, k, v, j * c, c, prompt)

        g = _graph(torch, ingest, 1)
        t = _time(torch, g, 2)
        pairs = prompt * (prompt + 1) // 2
        out.append({"chunk": c, "calls": calls, "ms": round(t, 3),
                    "tflops": round(4.0 * H * D * pairs / (t * 1e-3) / 1e12, 1),
                    "workgroups_per_call": A.attn_prefill_items(c)})
        print(f"[retune] prompt {prompt}, chunk {c}: {t:.3f} ms", file=sys.stderr, flush=True)
    return out


def sweep_min_tokens(torch, A, ctx, ns, max_splits=128):
    out = []
    gen = torch.Generator(device="cuda")
    gen.manual_seed(ctx + 1)
    nmax = max(ns)
    max_ctx = ctx + nmax
    w = _Weights(torch, gen, nmax)
    k = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
    v = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
    q = torch.empty(nmax * H * D, device="cuda")
    core = torch.empty(nmax * H * D, device="cuda")
    sc = A.DecodeScratch(max_splits)
    for n in ns:
        def by_decode(_i, n=n):
            for j in range(n):
                decode_call(A, w, q[:H * D], core[:H * D], k, v, sc, ctx + j + 1, max_ctx,
                            max_splits)

        def by_prefill(_i, n=n):
            prefill_call(A, w, q, core, k, v, ctx, n, max_ctx)

        td = _time(torch, _graph(torch, by_decode, 1), 4)
        tp = _time(torch, _graph(torch, by_prefill, 1), 4)
        out.append({"n": n, "decode_us": round(td * 1e3, 2), "prefill_us": round(tp * 1e3, 2),
                    "prefill_faster": bool(tp < td)})
        print(f"[retune] ctx {ctx}, n {n}: {n} decodes {td * 1e3:.1f} us, prefill "
              f"{tp * 1e3:.1f} us", file=sys.stderr, flush=True)
    first = next((r["n"] for r in out if r["prefill_faster"]), None)
    return {"ctx": ctx, "rows": out, "smallest_n_where_prefill_wins": first}


def sweep_prefill_map(torch, A, prefixes, sizes):
    out = []
    gen = torch.Generator(device="cuda")
    for pos0 in prefixes:
        for n in sizes:
            max_ctx = pos0 + n
            gen.manual_seed(max_ctx + 7)
            q = torch.randn(n * H * D, generator=gen, device="cuda")
            qg = torch.randn(n * H * 2 * D, generator=gen, device="cuda")
            k = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
            v = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
            core = torch.empty(n * H * D, device="cuda")
            g = _graph(torch, lambda _i: A.attn_prefill(q, qg, k, v, core, pos0, n, max_ctx), 1)
            t = _time(torch, g, 3)
            pairs = n * pos0 + n * (n + 1) // 2
            out.append({"pos0": pos0, "n": n, "workgroups": A.attn_prefill_items(n),
                        "ms": round(t, 4), "tflops": round(4.0 * H * D * pairs / (t * 1e-3) / 1e12, 1)})
            print(f"[retune] prefill pos0 {pos0} n {n}: {t:.3f} ms, {out[-1]['tflops']} TFLOP/s",
                  file=sys.stderr, flush=True)
            del q, qg, k, v, core, g
    return out


def run(quick=False):
    import torch
    from miso_amd import attention as A

    if not torch.cuda.is_available():
        raise RuntimeError("retune needs a GPU")
    if quick:
        contexts, prompt, chunks, ns, ctx = [512, 4096], 2048, [512, 2048], [1, 2, 4], 1024
    else:
        contexts = [512, 4096, 32768, 131072]
        prompt, chunks = 8192, [256, 512, 1024, 2048, 4096, 8192]
        ns, ctx = [1, 2, 3, 4, 6, 8, 12, 16], 4096
    prefixes, sizes = ([0, 4096], [256, 1024]) if quick else \
        ([0, 8192, 32768], [512, 1024, 2048, 4096, 8192, 16384])
    return {
        "engine_constants": {"kMaxSplits": 60, "kMaxChunk": 512, "kPrefillMinTokens": 8},
        "max_splits": sweep_max_splits(torch, A, contexts),
        "chunk": {"prompt": prompt, "rows": sweep_chunk(torch, A, prompt, chunks)},
        "min_tokens": sweep_min_tokens(torch, A, ctx, ns),
        "prefill_map": sweep_prefill_map(torch, A, prefixes, sizes),
        "note": "attention kernels only (prep, split, combine, prep_batch, prefill), HIP-event "
                "time of graph replays, median of 3; synthetic N(0,1) inputs",
    }


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--quick", action="store_true", help="small sweep (seconds)")
    args = ap.parse_args(argv)
    print(json.dumps(run(args.quick)), flush=True)


if __name__ == "__main__":
    main()
