#!/usr/bin/env python3
"""Benchmark of the MI355X attention path (one GPU), printing ONE JSON line.

Headline (BASELINE.json metric, config C2): decode attention for 1 sequence / 1 token at context
32768 (16 query heads, 2 KV heads, head_dim 256, f16 KV cache [2][32768][256], N(0,1) synthetic
inputs), split-K over the KV length + LSE merge x sigmoid gate, in the reference's arithmetic
(f32 query, scores, numerators and accumulation; the f16-query variant is a labelled
other_configs line). A step = one decode call
(split + combine kernels) over one KV cache; `value` = algorithmic KV bytes (67,108,864 B per
step) / measured time, in GB/s. The inputs are resident in HBM; steps rotate over 6 distinct KV
caches (384 MiB > the 256 MiB Infinity Cache) so every step streams from HBM.

Also reported:
  roofline      the split kernel (dominant) timed alone with HIP events on its stream:
                algorithmic bytes / average launch time vs the 8 TB/s HBM peak; `traffic` is the
                HBM bytes per launch from rocprofv3 FETCH_SIZE + WRITE_SIZE (profiles/), or null.
  prefill       C4: 8192 new tokens after an 8192-token prefix, causal, f16 MFMA; TFLOP/s over
                the unmasked (query, key) pairs (1.6493e12 FLOP) vs the 2516.6 TFLOP/s f16 peak.
  cpu_baseline  the FP64 oracle (a C restatement of the reference's host scalar attention) on a
                bounded sample of the same workload on this host's CPU, rank 0 only: single
                thread and all cores (<= 16), with the CPU model and thread counts; its first
                call also checks the bench's own timed C2 output (the bench exits 3 on a
                mismatch).
  other_configs C2_f16q (C2 with the f16-query variant), C2_engine_cap60 (C2 at the engine's
                shipped split capacity of 60), C1 (decode, ctx 512: us per call), C3 (prefill, 2048 tokens, empty cache:
                TFLOP/s), C5 (ragged decode, 64 sequences: GB/s of K/V), as in the survey's table,
                and C5 over a pool of 16-row KV pages (the paged entry point); C2 over an fp8
                (e4m3 rows) KV cache: us per decode step and GB/s of codes + row scales.
                F4_qgemm: the prefill projection GEMMs at a 4096-token chunk (TFLOP/s).
                F4_q4k_gemv / F4_q6k_gemv: the Q4_K and Q6_K GEMVs at the attention's projection
                shapes (us, GB/s of weights).
  device        clock / temperature / power readings (rocm-smi or amd-smi) right after the runs.

Decode steps are timed the way the reference's own bench times them (bench/attention/
bench_attention.hip:24-33): back-to-back eager calls of the C ABI on one stream between two HIP
events, from a native loop (miso_amd/lib/libmiso_bench.so), since a Python caller's per-call cost
is of the order of a step. The same calls recorded into a HIP graph and replayed are reported
beside them (`graph_*`): on this ROCm each graph kernel node costs ~1-2.5 us more than an eager
launch. Without the native loop the graph figures are the measurement.

    python bench.py [--gpus 1] [--steps 60] [--warmup 12]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

H, KV, D = 16, 2, 256
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2516.6
METRIC = "decode-attn HBM GB/s @32k ctx; prefill-attn TFLOP/s @8k; % of roofline"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=60)
    ap.add_argument("--warmup", type=int, default=12)
    ap.add_argument("--ctx", type=int, default=32768)
    ap.add_argument("--buffers", type=int, default=6)
    ap.add_argument("--max-splits", type=int, default=128)
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--prefill-steps", type=int, default=10)
    ap.add_argument("--no-other", action="store_true", help="skip the C1 / C3 / C5 lines")
    ap.add_argument("--other", default=None,
                    help="comma-separated subset of the other configurations: C2var (the C2 "
                         "variants: f16 query, VALU split, combine curve, fused, cap 60), C1, "
                         "C3, C5 (with C5_paged), fp8 (C2_fp8, C2_long, C4_fp8), gemv, qgemm, "
                         "layer")
    ap.add_argument("--split-valu", action="store_true",
                    help="with --no-other: still time the VALU form of the C2 split (for "
                         "counter runs of both split forms)")
    ap.add_argument("--no-device", action="store_true",
                    help="skip the rocm-smi / amd-smi readings (implied under a profiler)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 3 plain 64 MiB device copies (counter calibration for "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE passes)")
    return ap.parse_args()


def copy_calibration(torch):
    """Three device-to-device copies of exactly 64 MiB: the known-size reference that scales the
    FETCH_SIZE / WRITE_SIZE counters of the attention kernels to HBM bytes."""
    src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log("copy calibration: 3 x 64 MiB device copies")


def graph_of(torch, fn, count):
    """Record `count` calls fn(i) into a HIP graph (after one eager warm call per i)."""
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


def time_replays(torch, g, reps):
    """Wall and event time of `reps` replays of g on the current stream (ms total)."""
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record()
    for _ in range(reps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1), (time.perf_counter() - t0) * 1e3


def device_state():
    """A few clock / temperature / power readings from rocm-smi (or amd-smi), best effort."""
    import subprocess
    for cmd in (["rocm-smi", "--showtemp", "--showpower", "--showclocks", "--json"],
                ["amd-smi", "metric", "--json"]):
        try:
            res = subprocess.run(cmd, capture_output=True, text=True, timeout=30)
        except (OSError, subprocess.SubprocessError) as e:
            last = f"{cmd[0]}: {e}"
            continue
        if res.returncode != 0 or not res.stdout.strip():
            last = f"{cmd[0]}: rc {res.returncode} {res.stderr.strip()[:120]}"
            continue
        try:
            data = json.loads(res.stdout)
        except ValueError:
            return {"tool": cmd[0], "raw": res.stdout.strip()[:400]}
        keep = {}

        def walk(prefix, node):
            if isinstance(node, dict):
                for k, v in node.items():
                    walk(f"{prefix}{k}/", v)
            elif isinstance(node, list):
                for i, v in enumerate(node[:4]):
                    walk(f"{prefix}{i}/", v)
            elif any(w in prefix.lower() for w in ("sclk", "mclk", "fclk", "temp", "power",
                                                   "socket", "gfx_clk", "clk")):
                if len(keep) < 24:
                    keep[prefix.rstrip("/")] = node

        walk("", data)
        return {"tool": cmd[0], "readings": keep}
    return {"error": last}


def traffic_from_profiles(name):
    p = ROOT / "profiles" / f"{name}_traffic.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def decode_caches(torch, args):
    """C2 inputs: q, qg and `buffers` distinct N(0,1) f16 KV caches of ctx positions."""
    L, R = args.ctx, args.buffers
    gen = torch.Generator(device="cuda")
    gen.manual_seed(L)
    q = torch.randn(H * D, generator=gen, device="cuda")
    qg = torch.randn(H * 2 * D, generator=gen, device="cuda")
    caches = []
    for _ in range(R):
        k = torch.randn(KV * L * D, generator=gen, device="cuda").half()
        v = torch.randn(KV * L * D, generator=gen, device="cuda").half()
        caches.append((k, v))
    return q, qg, caches


def eager_loop():
    """The native eager timing loop (libmiso_bench.so), or None if it is not built."""
    import ctypes
    path = ROOT / "miso_amd" / "lib" / "libmiso_bench.so"
    if not path.exists():
        return None
    lib = ctypes.CDLL(str(path))
    vp, u32, i32 = ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int
    lib.miso_bench_decode.restype = ctypes.c_double
    lib.miso_bench_decode.argtypes = [i32, vp, vp, ctypes.POINTER(vp), ctypes.POINTER(vp), i32,
                                      vp, vp, vp, vp, u32, u32, u32, i32, i32, vp, vp]
    lib.miso_bench_layer_decode.restype = ctypes.c_double
    lib.miso_bench_layer_decode.argtypes = [vp, vp, vp, u32, u32, vp, vp, ctypes.c_float, vp, i32,
                                            vp]
    return lib


def bench_fused(torch, A, lib, args, inputs, dec):
    """The C2 step in one launch (miso_attn_decode_fused: the splits hand their partials to the
    last arrivals of each KV head through an agent-scope counter, which merge them) against the
    two-launch step above: eager (median of 3 windows) and as graph replays."""
    q, qg, caches = inputs
    L, R, n = args.ctx, args.buffers, dec["n_splits"]
    sc = A.DecodeScratch(args.max_splits)
    core = torch.empty(H * D, device="cuda")
    w = sorted(eager_decode(torch, lib, 5, q, qg, caches, core, sc, L, n, args.warmup,
                            dec["steps"]) for _ in range(3))
    g = graph_of(torch, lambda i: A.attn_decode(q, qg, caches[i % R][0], caches[i % R][1], core,
                                                sc, L, L, n, fused=True), R)
    time_replays(torch, g, 2)
    reps = max(1, (args.steps + R - 1) // R)
    tg = sorted(time_replays(torch, g, reps)[0] for _ in range(3))[1] / (reps * R)
    log(f"decode C2 single launch: eager {w[1] * 1e3:.2f} us, graph {tg * 1e3:.2f} us "
        f"(two launches: eager {dec['t_step_ms'] * 1e3:.2f}, graph "
        f"{dec['graph_ms']['step'] * 1e3:.2f} us)")
    return {"workload": "C2 step in one launch (miso_attn_decode_fused): partials stored "
                        "agent-coherently, the last 32 arrivals per KV head merge the 64 "
                        "(head, 64-dimension) tiles; measured alternative to split + combine",
            "us_per_step": round(w[1] * 1e3, 3), "eager_windows_us": [round(x * 1e3, 3) for x in w],
            "graph_us_per_step": round(tg * 1e3, 3),
            "two_launch_us_per_step": round(dec["t_step_ms"] * 1e3, 3),
            "two_launch_graph_us_per_step": round(dec["graph_ms"]["step"] * 1e3, 3),
            "gbs": round(dec["kv_bytes"] / (w[1] * 1e-3) / 1e9, 1)}


def bench_combine_curve(torch, A, lib, inputs):
    """The combine alone against the split count, as the reference's bench/attention/
    bench_combine.hip:15-67 measures it: partials m ~ 10 U(-1, 1), l ~ 1 + 16 |U(-1, 1)|,
    o ~ U(-1, 1), gate ~ U(-1, 1) (own generator), 300 untimed then 2000 timed back-to-back
    launches between two events, median of 3 runs; us per launch."""
    q, qg, caches = inputs
    gen = torch.Generator(device="cuda")
    gen.manual_seed(71)
    cap = 129
    u = lambda n: torch.rand(n, generator=gen, device="cuda") * 2 - 1
    m = u(2 * cap * 8) * 10
    l_ = 1 + u(2 * cap * 8).abs() * 16
    o = u(2 * cap * 8 * 256)
    g = u(16 * 512)
    core = torch.empty(H * D, device="cuda")
    sc = type("Partials", (), {"part_m": m, "part_l": l_, "part_o": o})()
    curve = {}
    for ns in (1, 16, 22, 57, 60, 65, 128, 129):
        runs = sorted(eager_decode(torch, lib, 2, q, g, caches[:1], core, sc, 0, ns, 300, 2000)
                      for _ in range(3))
        curve[str(ns)] = round(runs[1] * 1e3, 3)
    log(f"combine alone (us per launch by split count): {curve}")
    return {"workload": "attn_combine_kernel<64,true,4><<<64,64>>> alone over random partials, "
                        "by split count (the reference's bench/attention/bench_combine.hip "
                        "method: 300 warm + 2000 timed launches, median of 3 runs)",
            "us_by_splits": curve}


def eager_decode(torch, lib, mode, q, qg, caches, core, sc, L, n_splits, warmup, iters):
    """ms per call of `iters` eager calls (mode: 0 decode, 1 split, 2 combine, 3 decode f16q,
    4 split on VALU, 5 single-launch decode)."""
    import ctypes
    R = len(caches)
    ks = (ctypes.c_void_p * R)(*[k.data_ptr() for k, _ in caches])
    vs = (ctypes.c_void_p * R)(*[v.data_ptr() for _, v in caches])
    torch.cuda.synchronize()
    sync = getattr(sc, "sync", None)
    ms = lib.miso_bench_decode(mode, q.data_ptr(), qg.data_ptr(), ks, vs, R, core.data_ptr(),
                               sc.part_m.data_ptr(), sc.part_l.data_ptr(), sc.part_o.data_ptr(),
                               L, L, n_splits, warmup, iters,
                               torch.cuda.current_stream().cuda_stream,
                               sync.data_ptr() if sync is not None else None)
    if ms < 0:
        raise RuntimeError(f"eager timing loop failed ({ms})")
    return ms


def bench_decode(torch, A, args, inputs, max_splits, f16_query=False, label="C2"):
    """One decode call per step over rotated caches: step (split + combine), split alone and
    combine alone, each as a graph of `buffers` calls replayed; per-call times in ms. Returns
    the output of one call on cache 0 for the oracle check."""
    q, qg, caches = inputs
    L, R = args.ctx, args.buffers
    sc = A.DecodeScratch(max_splits)
    n_splits = A.attn_n_splits(L, max_splits)
    core = torch.empty(H * D, device="cuda")
    kv_bytes = 2 * KV * L * D * 2

    def step(i):
        k, v = caches[i % R]
        A.attn_decode(q, qg, k, v, core, sc, L, L, n_splits, f16_query=f16_query)

    def split_only(i):
        k, v = caches[i % R]
        if f16_query:
            A.attn_decode(q, qg, k, v, core, sc, L, L, n_splits, f16_query=True)
        else:
            A.attn_split(q, k, v, sc.part_m, sc.part_l, sc.part_o, L, L, n_splits)

    def combine_only(i):
        A.attn_combine(sc.part_m, sc.part_l, sc.part_o, qg, core, n_splits)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    reps = max(1, (args.steps + R - 1) // R)
    steps = reps * R
    g_step = graph_of(torch, step, R)
    g_split = graph_of(torch, split_only, R)
    g_comb = graph_of(torch, combine_only, R)
    time_replays(torch, g_step, 2)  # warm the graph path
    ms_step, wall_step = time_replays(torch, g_step, reps)
    ms_split, _ = time_replays(torch, g_split, reps)
    ms_comb, _ = time_replays(torch, g_comb, reps)
    g_step_t = ms_step / steps
    g_split_t = ms_split / steps
    g_comb_t = ms_comb / steps
    if f16_query:
        g_split_t -= g_comb_t  # the f16q graph above times split + combine
    log(f"decode {label} (graph): step {g_step_t * 1e3:.2f} us (wall "
        f"{wall_step / steps * 1e3:.2f} us), split {g_split_t * 1e3:.2f} us, combine "
        f"{g_comb_t * 1e3:.2f} us, n_splits {n_splits}")
    timing = "graph"
    t_step, t_split, t_comb = g_step_t, g_split_t, g_comb_t
    lib = eager_loop()
    windows = None
    if lib is not None:
        timing = "eager"
        windows = {}

        def ev(mode, name):
            # the median of three eager windows of `steps` calls each
            w = [eager_decode(torch, lib, mode, q, qg, caches, core, sc, L, n_splits, args.warmup,
                              steps) for _ in range(3)]
            windows[name] = [round(x * 1e3, 3) for x in w]
            return sorted(w)[1]

        t_step = ev(3 if f16_query else 0, "step")
        t_comb = ev(2, "combine")
        t_split = ev(1, "split") if not f16_query else t_step - t_comb
        log(f"decode {label} (eager, median of 3 windows): step {t_step * 1e3:.2f} us "
            f"{windows['step']}, split {t_split * 1e3:.2f} us, combine {t_comb * 1e3:.2f} us")
    step(0)
    torch.cuda.synchronize()
    return {
        "steps": steps, "t_step_ms": t_step, "t_split_ms": t_split, "t_comb_ms": t_comb,
        "graph_ms": {"step": g_step_t, "split": g_split_t, "combine": g_comb_t},
        "timing": timing, "windows_us": windows,
        "kv_bytes": kv_bytes, "n_splits": n_splits, "L": L, "core0": core.cpu().numpy(),
    }


def decode_line(dec, workload):
    gbs = dec["kv_bytes"] / (dec["t_step_ms"] * 1e-3) / 1e9
    return {"workload": workload, "us_per_step": round(dec["t_step_ms"] * 1e3, 3),
            "split_us": round(dec["t_split_ms"] * 1e3, 3),
            "combine_us": round(dec["t_comb_ms"] * 1e3, 3), "n_splits": dec["n_splits"],
            "timing": dec["timing"],
            "graph_us_per_step": round(dec["graph_ms"]["step"] * 1e3, 3),
            "eager_windows_us": dec["windows_us"],
            "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}


def bench_prefill(torch, A, args):
    pos0, n = 8192, 8192
    max_ctx = pos0 + n
    gen = torch.Generator(device="cuda")
    gen.manual_seed(max_ctx)
    q = torch.randn(n * H * D, generator=gen, device="cuda")
    qg = torch.randn(n * H * 2 * D, generator=gen, device="cuda")
    k = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
    v = torch.randn(KV * max_ctx * D, generator=gen, device="cuda").half()
    core = torch.empty(n * H * D, device="cuda")

    def call(_):
        A.attn_prefill(q, qg, k, v, core, pos0, n, max_ctx)

    call(0)
    torch.cuda.synchronize()
    g = graph_of(torch, call, 1)
    time_replays(torch, g, 1)
    runs = sorted(time_replays(torch, g, args.prefill_steps)[0] for _ in range(3))
    t = runs[1] / args.prefill_steps  # median of 3 timed runs
    pairs = n * pos0 + n * (n + 1) // 2
    flop = 4.0 * H * D * pairs
    tflops = flop / (t * 1e-3) / 1e12
    log(f"prefill C4: {t:.3f} ms, {tflops:.1f} TFLOP/s")
    host = None
    if not args.no_cpu:
        torch.cuda.synchronize()
        host = {
            "q": q.cpu().numpy(), "qg": qg.cpu().numpy(),
            "k": k.view(torch.int16).cpu().numpy().view("uint16"),
            "v": v.view(torch.int16).cpu().numpy().view("uint16"),
            "core": core.cpu().numpy().reshape(n, H, D),  # the last timed call's output
        }
    return {"t_ms": t, "flop": flop, "tflops": tflops, "pos0": pos0, "n": n,
            "max_ctx": max_ctx, "host": host}


def synthetic_q4k(torch, gen, copies, n, k):
    """copies x n rows of random Q4_K r1 blocks (uint8 [copies][n k / 256 x 144]) whose f16 d and
    dmin (bytes 0..3 of each block) are finite: d = 0.00598, dmin = 0.00296."""
    w = torch.randint(0, 256, (copies, n * k // 256 * 144), dtype=torch.uint8, device="cuda",
                      generator=gen)
    w.view(copies, -1, 144)[:, :, 0:4] = torch.tensor([0x1F, 0x1E, 0x0F, 0x1A], dtype=torch.uint8,
                                                      device="cuda")
    return w


def synthetic_q6k(torch, gen, copies, n, k):
    """copies x n random Q6_K r1 rows ([ql][qh][scales][d][padding] per row) with every d finite
    (0x1A00 = 0.00293) and the padding zero."""
    nb = k // 256
    row = (nb * 210 + 15) // 16 * 16
    w = torch.randint(0, 256, (copies, n, row), dtype=torch.uint8, device="cuda", generator=gen)
    w[:, :, nb * 208:] = 0
    w[:, :, nb * 208 + 1:nb * 210:2] = 0x1A  # the high byte of each f16 d
    return w.reshape(copies, -1)


def bench_other(torch, A, args):
    """The other configurations (synthetic N(0,1) inputs): C1, C3, C5 (contiguous and paged),
    C2 / C4 over an fp8 cache, the projection GEMVs and GEMMs, the layer step. --other picks a
    subset (for profiler runs)."""
    import numpy as np
    out = {}
    pick = None if args.other is None else set(args.other.split(","))

    def want(name):
        return pick is None or name in pick

    gen = torch.Generator(device="cuda")
    if want("C1"):
        # C1: decode at ctx 512 (1 MiB of K/V: cache-resident, latency-bound).
        L = 512
        gen.manual_seed(L)
        q = torch.randn(H * D, generator=gen, device="cuda")
        qg = torch.randn(H * 2 * D, generator=gen, device="cuda")
        k = torch.randn(KV * L * D, generator=gen, device="cuda").half()
        v = torch.randn(KV * L * D, generator=gen, device="cuda").half()
        sc = A.DecodeScratch(args.max_splits)
        n1 = A.attn_n_splits(L, args.max_splits)
        core = torch.empty(H * D, device="cuda")
        g = graph_of(torch, lambda i: A.attn_decode(q, qg, k, v, core, sc, L, L, n1), 6)
        time_replays(torch, g, 2)
        ms = sorted(time_replays(torch, g, 20)[0] for _ in range(3))[1]
        t1 = ms / 120
        out["C1"] = {"workload": "decode, 1 sequence x 1 token, ctx 512 (warm cache)",
                     "us_per_call": round(t1 * 1e3, 3), "n_splits": n1,
                     "gbs": round(2048 * L / (t1 * 1e-3) / 1e9, 1)}
    if want("C3"):
        # C3: causal prefill, 2048 tokens, empty cache.
        n3 = 2048
        gen.manual_seed(n3)
        q = torch.randn(n3 * H * D, generator=gen, device="cuda")
        qg = torch.randn(n3 * H * 2 * D, generator=gen, device="cuda")
        k = torch.randn(KV * n3 * D, generator=gen, device="cuda").half()
        v = torch.randn(KV * n3 * D, generator=gen, device="cuda").half()
        core = torch.empty(n3 * H * D, device="cuda")
        flop3 = 4.0 * H * D * (n3 * (n3 + 1) // 2)
        # Ten calls per graph (one call per replay is bound by the replay launch, ~89 us here), the
        # balanced form (miso_attn_prefill_ws) and the one-workgroup-per-block form side by side.
        scratch = A.PrefillScratch(n3)
        t3 = {}
        for form, sc in (("balanced", scratch), ("one_block", None)):
            g = graph_of(torch, lambda i: A.attn_prefill(q, qg, k, v, core, 0, n3, n3, scratch=sc), 10)
            time_replays(torch, g, 1)
            t3[form] = sorted(time_replays(torch, g, 2)[0] for _ in range(3))[1] / 20
            del g
        out["C3"] = {"workload": "causal prefill, 2048 tokens, empty cache (balanced form)",
                     "ms_per_call": round(t3["balanced"], 4),
                     "tflops": round(flop3 / (t3["balanced"] * 1e-3) / 1e12, 1),
                     "frac": round(flop3 / (t3["balanced"] * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                     "one_block_ms_per_call": round(t3["one_block"], 4),
                     "one_block_tflops": round(flop3 / (t3["one_block"] * 1e-3) / 1e12, 1)}
        del q, qg, k, v, core, scratch
    if want("C5"):
        # C5: ragged decode, 64 sequences, lengths uniform in [1024, 16384] (numpy, seed 64).
        lens = np.random.default_rng(64).integers(1024, 16385, 64).astype(np.int64)
        offs = np.zeros(64, dtype=np.int64)
        offs[1:] = np.cumsum(lens * KV * D)[:-1]
        total = int((lens * KV * D).sum())
        gen.manual_seed(64)
        qb = torch.randn(64 * H * D, generator=gen, device="cuda")
        gate = torch.randn(64 * H * D, generator=gen, device="cuda")
        kc = torch.randn(total, generator=gen, device="cuda").half()
        vc = torch.randn(total, generator=gen, device="cuda").half()
        d_offs = torch.from_numpy(offs).cuda()
        d_lens = torch.from_numpy(lens.astype(np.int32)).cuda()
        scr = A.RaggedScratch(64, int(lens.max()))
        core = torch.empty(64 * H * D, device="cuda")
        g = graph_of(torch, lambda i: A.attn_decode_ragged(qb, gate, kc, vc, d_offs, d_lens, core,
                                                           scr), 1)
        time_replays(torch, g, 2)
        ms = sorted(time_replays(torch, g, 10)[0] for _ in range(3))[1]
        t5 = ms / 10
        bytes5 = 2048.0 * float(lens.sum())
        out["C5"] = {"workload": "ragged decode, 64 sequences x 1 token, lengths U[1024,16384] "
                                 "(numpy seed 64), dense sigmoid gate",
                     "sum_len": int(lens.sum()), "ms_per_call": round(t5, 4),
                     "gbs": round(bytes5 / (t5 * 1e-3) / 1e9, 1),
                     "frac": round(bytes5 / (t5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del kc, vc
        # C5 over a KV page pool: the same lengths, 16-row pages in a random order.
        page = 16
        npg = (lens + page - 1) // page
        max_pages = int(npg.max())
        pool = int(npg.sum())
        perm = np.random.default_rng(65).permutation(pool).astype(np.int32)
        table = np.zeros((64, max_pages), np.int32)
        starts = np.concatenate([[0], np.cumsum(npg)[:-1]])
        for s_, (st, n_) in enumerate(zip(starts, npg)):
            table[s_, :n_] = perm[st:st + n_]
        kp = torch.randn(pool * KV * page * D, generator=gen, device="cuda").half()
        vp = torch.randn(pool * KV * page * D, generator=gen, device="cuda").half()
        d_table = torch.from_numpy(table).cuda()
        g = graph_of(torch, lambda i: A.attn_decode_paged(qb, gate, kp, vp, d_table, page, d_lens,
                                                          core, scr), 1)
        time_replays(torch, g, 2)
        ms = sorted(time_replays(torch, g, 10)[0] for _ in range(3))[1]
        t5p = ms / 10
        out["C5_paged"] = {"workload": "C5 with the K/V in a pool of 16-row pages in a random order "
                                       "(page table per sequence)",
                           "page_size": page, "pages": pool, "ms_per_call": round(t5p, 4),
                           "gbs": round(bytes5 / (t5p * 1e-3) / 1e9, 1),
                           "frac": round(bytes5 / (t5p * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del kp, vp
    if want("fp8"):
        # C2 over an fp8 (e4m3 rows) cache: the same context and buffer rotation as the C2 line,
        # each cache encoded on the GPU from an N(0,1) f16 cache.
        L, R = args.ctx, args.buffers
        gen.manual_seed(L + 1)
        q = torch.randn(H * D, generator=gen, device="cuda")
        qg = torch.randn(H * 2 * D, generator=gen, device="cuda")
        caches8 = []
        for _ in range(R):
            k = torch.randn(KV * L * D, generator=gen, device="cuda").half()
            v = torch.randn(KV * L * D, generator=gen, device="cuda").half()
            c8 = A.Fp8Cache(L)
            A.attn_kv_encode_fp8(k, v, c8, 0, L)
            caches8.append(c8)
        del k, v
        sc = A.DecodeScratch(args.max_splits)
        n8 = A.attn_n_splits(L, args.max_splits)
        core = torch.empty(H * D, device="cuda")
        g = graph_of(torch, lambda i: A.attn_decode_fp8(q, qg, caches8[i % R], core, sc, L, n8), R)
        time_replays(torch, g, 2)
        reps = max(1, (args.steps + R - 1) // R)
        ms = sorted(time_replays(torch, g, reps)[0] for _ in range(3))[1]
        t8 = ms / (reps * R)
        bytes8 = 2.0 * KV * L * (D + 4)  # codes and row scales of K and V
        out["C2_fp8"] = {"workload": f"C2 (decode, 1 sequence x 1 token, ctx {L}) over an e4m3-row "
                                     "KV cache (1-byte codes + one f32 scale per row)",
                         "us_per_step": round(t8 * 1e3, 2), "n_splits": n8,
                         "kv_bytes": int(bytes8), "gbs": round(bytes8 / (t8 * 1e-3) / 1e9, 1),
                         "frac": round(bytes8 / (t8 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        del caches8
        # Decode where the stream is long: 262144 keys (the engine's largest cache), the f16 and
        # the e4m3-row cache side by side, 128 splits, two rotated caches each.
        Lg = 262144
        gen.manual_seed(Lg)
        lk = [torch.randn(KV * Lg * D, generator=gen, device="cuda").half() for _ in range(4)]
        long16 = [(lk[0], lk[1]), (lk[2], lk[3])]
        long8 = []
        for kk, vv in long16:
            c8 = A.Fp8Cache(Lg)
            A.attn_kv_encode_fp8(kk, vv, c8, 0, Lg)
            long8.append(c8)
        nl = A.attn_n_splits(Lg, args.max_splits)
        g = graph_of(torch, lambda i: A.attn_decode(q, qg, long16[i % 2][0], long16[i % 2][1],
                                                    core, sc, Lg, Lg, nl), 2)
        time_replays(torch, g, 2)
        tl16 = sorted(time_replays(torch, g, 10)[0] for _ in range(3))[1] / 20
        del g
        g = graph_of(torch, lambda i: A.attn_decode_fp8(q, qg, long8[i % 2], core, sc, Lg, nl), 2)
        time_replays(torch, g, 2)
        tl8 = sorted(time_replays(torch, g, 10)[0] for _ in range(3))[1] / 20
        del g, lk, long16, long8
        out["C2_long"] = {"workload": f"decode, 1 sequence x 1 token, ctx {Lg}, over the f16 and "
                                      "the e4m3-row cache (graph replays)",
                          "n_splits": nl, "f16_us_per_step": round(tl16 * 1e3, 2),
                          "f16_gbs": round(2048.0 * Lg / (tl16 * 1e-3) / 1e9, 1),
                          "fp8_us_per_step": round(tl8 * 1e3, 2),
                          "fp8_gbs": round(2.0 * KV * Lg * (D + 4) / (tl8 * 1e-3) / 1e9, 1)}
        # C4 over an e4m3-row cache: the 16384 rows widened to f16 into a workspace each call, then
        # the f16 prefill (attn_prefill_fp8).
        if not args.no_prefill:
            pos0, n = 8192, 8192
            m4 = pos0 + n
            gen.manual_seed(m4 + 1)
            q4 = torch.randn(n * H * D, generator=gen, device="cuda")
            qg4 = torch.randn(n * H * 2 * D, generator=gen, device="cuda")
            c8 = A.Fp8Cache(m4)
            A.attn_kv_encode_fp8(torch.randn(KV * m4 * D, generator=gen, device="cuda").half(),
                                 torch.randn(KV * m4 * D, generator=gen, device="cuda").half(),
                                 c8, 0, m4)
            ws4 = A.Fp8PrefillScratch(m4)
            core4 = torch.empty(n * H * D, device="cuda")
            g = graph_of(torch, lambda _: A.attn_prefill_fp8(q4, qg4, c8, core4, pos0, n, ws4), 1)
            time_replays(torch, g, 1)
            t4 = sorted(time_replays(torch, g, args.prefill_steps)[0]
                        for _ in range(3))[1] / args.prefill_steps
            flop4 = 4.0 * H * D * (n * pos0 + n * (n + 1) // 2)
            out["C4_fp8"] = {"workload": "C4 (causal prefill, 8192 tokens after an 8192-token prefix) "
                                         "over an e4m3-row cache: rows widened to f16, then the f16 "
                                         "prefill",
                             "ms_per_call": round(t4, 4),
                             "tflops": round(flop4 / (t4 * 1e-3) / 1e12, 1)}
            del c8, ws4, q4, qg4, core4
    if want("gemv"):
        # The projection GEMVs (row f4), f16 activations as the engine; weights rotated over >= 512 MB
        # of copies so they stream from HBM as a model's layers do.
        def rotated(nbytes):
            return max(2, -(-(512 << 20) // nbytes))

        def timed(fn, copies):
            g = graph_of(torch, fn, copies)
            time_replays(torch, g, 1)
            return sorted(time_replays(torch, g, 3)[0] for _ in range(3))[1] / (3 * copies)

        def line(wbytes, t, copies, **extra):
            return {**extra, "weight_bytes": wbytes, "us_per_call": round(t * 1e3, 2),
                    "gbs": round(wbytes / (t * 1e-3) / 1e9, 1),
                    "frac": round(wbytes / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "weight_copies_rotated": copies}

        x2048 = torch.randn(2048, generator=gen, device="cuda")
        x4096 = torch.randn(4096, generator=gen, device="cuda")
        gemv = {}
        for name, k, n in (("attn_q", 2048, 8192), ("attn_k", 2048, 512), ("attn_output", 4096, 2048)):
            wbytes = n * k // 256 * 144
            copies = rotated(wbytes)
            wq = synthetic_q4k(torch, gen, copies, n, k)
            yg = torch.empty(n, device="cuda")
            xg = x2048 if k == 2048 else x4096
            t = timed(lambda i: A.q4k_gemv(wq[i % copies], xg, yg, n, k), copies)
            gemv[name] = line(wbytes, t, copies, k=k, n_rows=n)
            del wq
        out["F4_q4k_gemv"] = {"workload": "Q4_K r1 GEMV y = W x with f16 activations at the engine's "
                                          "Q4_K attention projections (synthetic blocks, HBM-resident "
                                          "weights)", **gemv}
        # attn_v is Q6_K (2048 -> 512); the engine's gemv_pair runs it with attn_q in one launch.
        w6b, w4b = 512 * A.q6k_row_bytes(2048), 8192 * 2048 // 256 * 144
        copies = rotated(w6b)
        w6 = synthetic_q6k(torch, gen, copies, 512, 2048)
        y6 = torch.empty(512, device="cuda")
        t6 = timed(lambda i: A.q6k_gemv(w6[i % copies], x2048, y6, 512, 2048), copies)
        del w6
        copies_p = rotated(w4b + w6b)
        w4 = synthetic_q4k(torch, gen, copies_p, 8192, 2048)
        w6 = synthetic_q6k(torch, gen, copies_p, 512, 2048)
        y4 = torch.empty(8192, device="cuda")
        tp = timed(lambda i: A.q4k_q6k_gemv_pair(w4[i % copies_p], 8192, y4, w6[i % copies_p], 512, y6,
                                                 x2048), copies_p)
        wk = synthetic_q4k(torch, gen, copies_p, 512, 2048)
        yk = torch.empty(512, device="cuda")
        tq = timed(lambda i: A.qkv_gemv(w4[i % copies_p], 8192, y4, wk[i % copies_p], 512, yk,
                                        w6[i % copies_p], 512, y6, x2048), copies_p)
        del w4, w6, wk
        out["F4_q6k_gemv"] = {"workload": "Q6_K r1 GEMV, f16 activations, attn_v, alone and paired "
                                          "with attn_q in one launch (synthetic blocks, HBM-resident "
                                          "weights)",
                              "attn_v": line(w6b, t6, copies, k=2048, n_rows=512),
                              "attn_q_plus_attn_v_pair": line(w4b + w6b, tp, copies_p),
                              "attn_q_k_v_one_launch": line(w4b + w6b + 512 * 2048 // 256 * 144, tq,
                                                            copies_p)}
    if want("qgemm"):
        # Prefill projection GEMMs (row f4, kernels/qgemm.hpp) at a 4096-token chunk (the layer's
        # retuned prefill chunk): TFLOP/s of 2 n_tok n k over the dequantized product.
        n_tok = 4096
        gemm = {}
        for name, fmt, k, n in (("attn_q", "q4_k", 2048, 8192), ("attn_k", "q4_k", 2048, 512),
                                ("attn_v", "q6_k", 2048, 512), ("attn_output", "q4_k", 4096, 2048)):
            xa = torch.randn(n_tok * k, generator=gen, device="cuda")
            inp = A.GemmInput(n_tok, k)
            A.gemm_input(xa, k, n_tok, inp)
            wg = (synthetic_q4k(torch, gen, 1, n, k) if fmt == "q4_k"
                  else synthetic_q6k(torch, gen, 1, n, k))[0]
            ya = torch.empty(n_tok * n, device="cuda")
            tg = timed(lambda i: A.gemm(wg, fmt, n, k, inp, ya, n), 4)
            ta = timed(lambda i: A.gemm_input(xa, k, n_tok, inp), 4)
            fl = 2.0 * n_tok * n * k
            gemm[name] = {"format": fmt, "k": k, "n_rows": n, "us_per_call": round(tg * 1e3, 2),
                          "tflops": round(fl / (tg * 1e-3) / 1e12, 1),
                          "frac": round(fl / (tg * 1e-3) / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
                          "gemm_input_us": round(ta * 1e3, 2)}
            del xa, inp, wg, ya
        out["F4_qgemm"] = {"workload": f"prefill projection GEMMs over Q4_K / Q6_K r1 weights, "
                                       f"{n_tok} tokens, f16 activations (gemm_input) and f16 MFMA "
                                       f"with f32 accumulation; TFLOP/s of 2 n_tok n k",
                           "tokens": n_tok, **gemm}
    if want("layer"):
        # Row f3: one attention layer step through the engine wiring (miso_attn_layer_*), synthetic
        # Q4_K (q, k, o) and Q6_K (v) weights of the engine's shapes.
        gen.manual_seed(33)
        layer = A.Layer((synthetic_q4k(torch, gen, 1, 8192, 2048)[0], "q4_k"),
                        (synthetic_q4k(torch, gen, 1, 512, 2048)[0], "q4_k"),
                        (synthetic_q6k(torch, gen, 1, 512, 2048)[0], "q6_k"),
                        (synthetic_q4k(torch, gen, 1, 2048, 4096)[0], "q4_k"),
                        torch.ones(2048, device="cuda"), torch.ones(D, device="cuda"),
                        torch.ones(D, device="cuda"),
                        (1e7 ** (-torch.arange(32, device="cuda") / 32.0)).float())
        lws = A.LayerWorkspace(4096)
        Ld = 32768
        lk = torch.randn(KV * Ld * D, generator=gen, device="cuda").half()
        lv = torch.randn(KV * Ld * D, generator=gen, device="cuda").half()
        h = torch.randn(2048, generator=gen, device="cuda")
        dl = torch.randn(2048, generator=gen, device="cuda") * 0.1
        y = torch.empty(2048, device="cuda")
        g = graph_of(torch, lambda _: A.layer_decode(layer, lk, lv, Ld, Ld - 1, h, dl, y, 1e-6, lws),
                     1)
        time_replays(torch, g, 2)
        tl = sorted(time_replays(torch, g, 20)[0] for _ in range(3))[1] / 20
        ntk, p0 = 4096, 8192
        hp = torch.randn(ntk * 2048, generator=gen, device="cuda")
        yp = torch.empty(ntk * 2048, device="cuda")
        g = graph_of(torch, lambda _: A.layer_prefill(layer, lk, lv, Ld, p0, ntk, hp, None, yp, 1e-6,
                                                      lws), 1)
        time_replays(torch, g, 1)
        tp = sorted(time_replays(torch, g, 3)[0] for _ in range(3))[1] / 3
        curve = None
        lib = eager_loop()
        if lib is not None:
            # The reference's layer decode curve (bench/attention/bench_attention.hip:15-33): 64
            # eager decode steps between two events at each context, the cache growing by one row
            # per step, in a cache of 32768 + 256 rows; the median of 3 windows.
            import ctypes
            mc = 32768 + 256
            ck = torch.randn(KV * mc * D, generator=gen, device="cuda").half()
            cv = torch.randn(KV * mc * D, generator=gen, device="cuda").half()
            h1 = torch.full((2048,), 0.1, device="cuda")
            curve = {}
            for ctx in (16, 1024, 4096, 16384, 32768):
                w = []
                for _ in range(3):
                    torch.cuda.synchronize()
                    r = lib.miso_bench_layer_decode(
                        ctypes.addressof(layer.c), ck.data_ptr(), cv.data_ptr(), ctx, mc,
                        h1.data_ptr(), y.data_ptr(), 1e-6, lws.decode.data_ptr(), 64,
                        torch.cuda.current_stream().cuda_stream)
                    if r < 0:
                        raise RuntimeError(f"layer decode timing loop failed ({r})")
                    w.append(r)
                curve[str(ctx)] = round(sorted(w)[1] * 1e3, 2)
            del ck, cv
            log(f"layer decode curve (us per token, eager): {curve}")
        out["F3_layer"] = {"workload": "one attention layer step through the engine wiring "
                                       "(miso_attn_layer_decode / _prefill): residual + RMSNorm, "
                                       "q/k/v projections, prep, attention, output projection; "
                                       "synthetic Q4_K / Q6_K weights of the engine's shapes",
                           "decode_ctx": Ld, "decode_us_per_step": round(tl * 1e3, 2),
                           "decode_curve_us_per_token": curve,
                           "decode_curve_method": "the reference's bench/attention/"
                                                  "bench_attention.hip: 64 eager steps per context "
                                                  "between two events, cache growing; median of 3",
                           "prefill_tokens": ntk, "prefill_pos0": p0,
                           "prefill_ms_per_chunk": round(tp, 3)}
        del layer, lws, lk, lv, hp, yp
    log("other configurations: " + ", ".join(sorted(out)))
    return out


def cpu_info():
    """The host CPU as the box reports it: model name, std::thread::hardware_concurrency()'s
    equivalent (logical CPUs) and the CPUs this process may run on."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"model": model, "hardware_concurrency": os.cpu_count(), "usable_cpus": usable}


def cpu_threads():
    """All-core thread count for the oracle: the usable CPUs, at most 16 (the box's CPU share
    per GPU)."""
    return max(1, min(16, cpu_info()["usable_cpus"] or 1))


def cpu_decode_baseline(dec, inputs):
    """FP64 oracle on full C2 calls over the bench's first KV cache: single-thread (the
    reference's loops) for ~10 s, then all cores for ~5 s. The first call's output is also the
    check of the bench's own timed kernels: the step output on cache 0 must match it within the
    north star's tolerance and the reference's per-head rel-L2 gate, or the bench fails."""
    from oracle import oracle as O
    q, qg, caches = inputs
    h = {"q": q.cpu().numpy(), "qg": qg.cpu().numpy(),
         "k": caches[0][0].view(torch_mod().int16).cpu().numpy().view("uint16"),
         "v": caches[0][1].view(torch_mod().int16).cpu().numpy().view("uint16")}
    L = dec["L"]

    def timed(threads, budget, cap):
        reps, t0, out = 0, time.perf_counter(), None
        while True:
            r = O.decode_f64(h["q"], h["qg"], h["k"], h["v"], L, L, threads=threads)
            out = r if out is None else out
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget or reps >= cap:
                return reps, el, out

    reps1, el1, ref = timed(1, 10.0, 40)
    st = O.compare(dec["core0"].reshape(H, D), ref)
    check = {"max_abs": st["max_abs"], "rel_l2_head": st["rel_l2_head"], "ok": bool(
        st["ok"] and st["rel_l2_head"] <= 1e-5)}
    if not check["ok"]:
        print(f"bench.py: the timed C2 decode output disagrees with the FP64 oracle: {st}",
              file=sys.stderr, flush=True)
        sys.exit(3)
    nt = cpu_threads()
    repsn, eln, _ = timed(nt, 5.0, 400)
    single = dec["kv_bytes"] * reps1 / el1 / 1e9
    multi = dec["kv_bytes"] * repsn / eln / 1e9
    return {
        "value": single, "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"C2 decode (ctx 32768): {reps1} full FP64 oracle calls on KV cache 0, "
                  f"{el1:.1f} s, single thread (the reference's host loops); all-core line below",
        "ms_per_call": el1 / reps1 * 1e3,
        "all_cores": {"value": multi, "unit": "GB/s", "cores": nt,
                      "ms_per_call": eln / repsn * 1e3,
                      "sample": f"{repsn} full C2 oracle calls, {eln:.1f} s, {nt} threads over "
                                "the 16 heads"},
        "cpu": cpu_info(),
        "gpu_output_check": check,
    }


def torch_mod():
    import torch
    return torch


def cpu_prefill_baseline(pre):
    """FP64 oracle on a deterministic sample of C4 query rows (16 heads each), 16 threads:
    batches of 64 rows spread over the 8192 tokens until about 10 s of CPU work. Every oracle row
    is also the check of the bench's own timed C4 output: the sampled rows must match it within
    the north star's tolerance, or the bench fails (exit 3)."""
    import numpy as np
    from oracle import oracle as O
    h = pre["host"]
    threads = cpu_threads()
    order = np.arange(pre["n"], dtype=np.uint32)
    order = order[np.argsort((order * 2654435761) % pre["n"], kind="stable")]  # spread, fixed
    done, flop, t0, el = 0, 0.0, time.perf_counter(), 0.0
    worst = {"max_abs": 0.0, "max_rel": 0.0, "rel_l2_head": 0.0, "n_bad": 0}
    while done < order.size:
        rows = np.sort(order[done:done + 64])
        t1 = time.perf_counter()
        ref = O.prefill_f64(h["q"], h["qg"], H * 2 * D, h["k"], h["v"], pre["pos0"],
                            pre["max_ctx"], rows, threads=threads)
        el += time.perf_counter() - t1
        st = O.compare(h["core"][rows], ref)
        for key in worst:
            worst[key] = max(worst[key], st[key])
        if not st["ok"]:
            print(f"bench.py: the timed C4 prefill output disagrees with the FP64 oracle on rows "
                  f"{rows[:4]}...: {st}", file=sys.stderr, flush=True)
            sys.exit(3)
        flop += float(sum(4.0 * H * D * (pre["pos0"] + int(t) + 1) for t in rows))
        done += rows.size
        if time.perf_counter() - t0 >= 10.0:
            break
    return {"value": flop / el / 1e12, "unit": "TFLOP/s", "cores": threads, "kind": "port",
            "sample": f"C4 prefill: {done} query rows x 16 heads of the FP64 oracle (spread over "
                      f"the 8192 tokens), {el:.1f} s on {threads} threads",
            "gpu_output_check": {"rows": done, "ok": True, **worst}}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py: this build measures one GPU only (the attention path runs on a single "
              f"MI355X; multi-GPU sharding is a design note, not a bench line). Got --gpus "
              f"{args.gpus}, WORLD_SIZE {world}.", file=sys.stderr)
        sys.exit(2)
    import torch
    from miso_amd import attention as A

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    log(f"device: {torch.cuda.get_device_name(0)}")
    if args.copy_calibration:
        copy_calibration(torch)
    inputs = decode_caches(torch, args)
    dec = bench_decode(torch, A, args, inputs, args.max_splits)
    other = {}
    if args.no_other and args.split_valu and eager_loop() is not None:
        q, qg, caches = inputs
        sc = A.DecodeScratch(args.max_splits)
        core = torch.empty(H * D, device="cuda")
        t_valu = eager_decode(torch, eager_loop(), 4, q, qg, caches, core, sc, args.ctx,
                              dec["n_splits"], args.warmup, dec["steps"])
        log(f"decode C2 split on VALU (eager): {t_valu * 1e3:.2f} us")
    if not args.no_other and (args.other is None or "C2var" in args.other.split(",")):
        d16 = bench_decode(torch, A, args, inputs, args.max_splits, f16_query=True,
                           label="C2 f16 query")
        other["C2_f16q"] = decode_line(
            d16, "C2 with an f16 query and f16 numerators (v_dot2_f32_f16; miso_attn_decode_f16q):"
                 " half the VALU work, per-head rel-L2 ~3e-4 -- not the reference's arithmetic")
        lib = eager_loop()
        if lib is not None:
            q, qg, caches = inputs
            sc = A.DecodeScratch(args.max_splits)
            core = torch.empty(H * D, device="cuda")
            t_valu = eager_decode(torch, lib, 4, q, qg, caches, core, sc, args.ctx,
                                  dec["n_splits"], args.warmup, dec["steps"])
            log(f"decode C2 split on VALU (eager): {t_valu * 1e3:.2f} us")
            other["C2_split_valu"] = {
                "workload": "the C2 split alone computed on wave64 VALU (v_fma_mix_f32, one f32 "
                            "product per instruction; miso_attn_split_valu) instead of the matrix "
                            "cores, same precision and partials: the measured alternative",
                "split_us": round(t_valu * 1e3, 3),
                "mfma_split_us": round(dec["t_split_ms"] * 1e3, 3),
                "gbs": round(dec["kv_bytes"] / (t_valu * 1e-3) / 1e9, 1)}
            other["C2_combine_by_splits"] = bench_combine_curve(torch, A, lib, inputs)
            other["C2_fused"] = bench_fused(torch, A, lib, args, inputs, dec)
        d60 = bench_decode(torch, A, args, inputs, 60, label="C2 engine cap 60")
        other["C2_engine_cap60"] = decode_line(
            d60, "C2 at the engine's shipped partial capacity kMaxSplits = 60 "
                 "(src/engine/attention.hpp:46): 60 splits x 2 KV heads = 120 workgroups")
    pre = None if args.no_prefill else bench_prefill(torch, A, args)
    if not args.no_other:
        other.update(bench_other(torch, A, args))
    else:
        other = None
    # Right after the GPU runs, while the clocks are still up. Not under a profiler: its preloaded
    # library would initialise the GPU in the smi tools too, before they exec their interpreter.
    profiled = "rocprof" in os.environ.get("LD_PRELOAD", "")
    device = None if (args.no_device or profiled) else device_state()

    value = dec["kv_bytes"] / (dec["t_step_ms"] * 1e-3) / 1e9
    split_gbs = dec["kv_bytes"] / (dec["t_split_ms"] * 1e-3) / 1e9
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": dec["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(dec["t_step_ms"], 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "C2: decode attention, 1 sequence x 1 token, ctx 32768, 16Q/2KV heads, "
                        "head_dim 256, f16 KV [2][32768][256], split-K + LSE merge x sigmoid gate",
            "ctx": dec["L"], "n_splits": dec["n_splits"], "kv_buffers_rotated": args.buffers,
            "step": "split kernel + combine kernel (one decode call)",
            "timing": dec["timing"] + (" (native loop of eager C ABI calls between two HIP "
                                       "events, as bench/attention/bench_attention.hip; the "
                                       "median of 3 windows)"
                                       if dec["timing"] == "eager" else " (HIP graph replays)"),
            "graph_us_per_step": round(dec["graph_ms"]["step"] * 1e3, 3),
            "eager_windows_us": dec["windows_us"],
            "arithmetic": "the reference's precision (kernels/attention_decode.hpp:150-221): f32 "
                          "query and softmax numerators, each carried as an exact f16 (hi, lo) "
                          "pair into v_mfma_f32_16x16x32_f16 against the f16 KV cache, f32 "
                          "scores and accumulation; storage f16",
            "algorithmic_bytes_per_step": dec["kv_bytes"],
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "attn_split_kernel<256>",
            "achieved": round(split_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(split_gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic_from_profiles("decode_c2"),
            "avg_launch_us": round(dec["t_split_ms"] * 1e3, 3),
            "combine_avg_launch_us": round(dec["t_comb_ms"] * 1e3, 3),
            "step_frac": round(value / HBM_PEAK_GBS, 4),
        },
    }
    if pre is not None:
        out["prefill"] = {
            "workload": "C4: causal prefill, 8192 tokens after an 8192-token prefix (16384 keys), "
                        "16Q/2KV, head_dim 256, f16 MFMA, f32 softmax/accumulate",
            "value": round(pre["tflops"], 2), "unit": "TFLOP/s", "ms_per_call": round(pre["t_ms"], 4),
            "algorithmic_flop": pre["flop"],
            "roofline": {"bound": "mfma", "kernel": "attn_prefill_kernel<256>",
                         "achieved": round(pre["tflops"], 2), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(pre["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                         "traffic": traffic_from_profiles("prefill_c4")},
        }
    if other is not None:
        out["other_configs"] = other
    if device is not None:
        out["device"] = device
    if not args.no_cpu:
        log("cpu baseline (decode) ...")
        out["cpu_baseline"] = cpu_decode_baseline(dec, inputs)
        if pre is not None and pre["host"] is not None:
            log("cpu baseline (prefill sample) ...")
            out["prefill"]["cpu_baseline"] = cpu_prefill_baseline(pre)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
