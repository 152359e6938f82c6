"""One attention layer step in the engine's order (row f3: the host wiring of attention_decode /
attention_prefill, src/engine/attention.hip:76-148, with the retuned sizing) on MI355X through the
C ABI, against the float64 layer oracle (oracle.layer_f64: RMSNorm, the projections over the
dequantized rows with f16 activations as the reference's GEMV / GEMM take them, prep, attention
over the growing cache, output projection).

A sequence of calls exercises every path and the policy: ingest of 40 tokens in chunks of 16
(prefill 16, 16, 8), ingest of 5 tokens (below the threshold: 5 decode steps), ingest of 13 (one
prefill), a direct decode step and a direct 3-token prefill. Every token's y, the residual update
and the f16 KV cache are compared. Gates: decode tokens rel-L2 <= 1e-3 per token, prefill tokens
<= 5e-3 (the prefill attention's f16 MFMA arithmetic); h bit-exact (one f32 add); each K/V cache
entry within one f16 ulp of its value plus 1e-4 of its row's largest magnitude (both sides round
f32 values that differ only by accumulation order).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import to_dev, to_host

pytestmark = pytest.mark.gpu

MAX_CTX, EPS = 96, 1e-6


def q4k_blocks(rng, n, k):
    nb = n * k // 256
    b = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
    b[:, 0:2] = (rng.random(nb) * 4e-4 + 1e-4).astype(np.float16).view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = (rng.random(nb) * 1e-4 + 1e-5).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def q6k_blocks(rng, n, k):
    nb = n * k // 256
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    b[:, 208:210] = (rng.random(nb) * 2e-4 + 5e-5).astype(np.float16).view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


@pytest.fixture(scope="module")
def layer_case(O, attn, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(2026)
    blocks = {"q": q4k_blocks(rng, 8192, 2048), "k": q4k_blocks(rng, 512, 2048),
              "v": q6k_blocks(rng, 512, 2048), "o": q4k_blocks(rng, 2048, 4096)}
    dev = {"q": (to_dev(torch, O.q4k_repack_r1(blocks["q"])), "q4_k"),
           "k": (to_dev(torch, O.q4k_repack_r1(blocks["k"])), "q4_k"),
           "v": (to_dev(torch, O.q6k_repack_r1(blocks["v"], 512, 2048)), "q6_k"),
           "o": (to_dev(torch, O.q4k_repack_r1(blocks["o"])), "q4_k")}
    deq = {"q": O.q4k_dequant(blocks["q"])[0].reshape(8192, 2048),
           "k": O.q4k_dequant(blocks["k"])[0].reshape(512, 2048),
           "v": O.q6k_dequant(blocks["v"]).reshape(512, 2048),
           "o": O.q4k_dequant(blocks["o"])[0].reshape(2048, 4096)}
    norms = {"attn_norm": (1 + 0.1 * rng.standard_normal(2048)).astype(np.float32),
             "q_norm": (1 + 0.1 * rng.standard_normal(256)).astype(np.float32),
             "k_norm": (1 + 0.1 * rng.standard_normal(256)).astype(np.float32),
             "inv_freq": O.inv_freq(1e7)}
    layer = attn.Layer(dev["q"], dev["k"], dev["v"], dev["o"],
                       *(to_dev(torch, norms[k]) for k in ("attn_norm", "q_norm", "k_norm",
                                                           "inv_freq")))
    return layer, deq, norms


def test_layer_engine_order(O, attn, torch_mod, layer_case):
    torch = torch_mod
    layer, deq, norms = layer_case
    rng = np.random.default_rng(7)
    total = 40 + 5 + 13 + 1 + 3
    h0 = rng.standard_normal((total, 2048)).astype(np.float32)
    delta = (0.5 * rng.standard_normal((total, 2048))).astype(np.float32)
    h = to_dev(torch, h0.reshape(-1))
    d = to_dev(torch, delta.reshape(-1))
    y = torch.full((total * 2048,), -1234.5, dtype=torch.float32, device="cuda")
    kc = torch.zeros(2 * MAX_CTX * 256, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    ws = attn.LayerWorkspace(max_tok=16)

    def rows(t, a, b):
        return t[a * 2048:b * 2048]

    # (kind, first token, count, chunk); prefill tokens are those that went through a prefill
    calls = [("ingest", 0, 40, 16), ("ingest", 40, 5, 0), ("ingest", 45, 13, 0),
             ("decode", 58, 1, 0), ("prefill", 59, 3, 0)]
    prefilled = np.zeros(total, bool)
    for kind, a, n, chunk in calls:
        b = a + n
        if kind == "ingest":
            attn.layer_ingest(layer, kc, vc, MAX_CTX, a, n, rows(h, a, b), rows(d, a, b),
                              rows(y, a, b), EPS, ws, chunk=chunk)
            prefilled[a:b] = n >= attn.LAYER_PREFILL_MIN_TOKENS
        elif kind == "decode":
            attn.layer_decode(layer, kc, vc, MAX_CTX, a, rows(h, a, b), rows(d, a, b),
                              rows(y, a, b), EPS, ws)
        else:
            attn.layer_prefill(layer, kc, vc, MAX_CTX, a, n, rows(h, a, b), rows(d, a, b),
                               rows(y, a, b), EPS, ws)
            prefilled[a:b] = True
    torch.cuda.synchronize()

    ref_h, ref_y, k16, v16 = O.layer_f64(h0, delta, deq["q"], deq["k"], deq["v"], deq["o"],
                                         norms["attn_norm"], norms["q_norm"], norms["k_norm"],
                                         norms["inv_freq"], 0, MAX_CTX, EPS)
    got_h = to_host(h).reshape(total, 2048)
    assert np.array_equal(got_h, ref_h), "residual update"
    got_y = to_host(y).reshape(total, 2048).astype(np.float64)
    err = np.sqrt(((got_y - ref_y) ** 2).sum(axis=1) / (ref_y ** 2).sum(axis=1))
    print(f"[layer] decode tokens max rel-L2 {err[~prefilled].max():.2e}, prefill tokens "
          f"{err[prefilled].max():.2e}", flush=True)
    assert np.isfinite(got_y).all()
    assert err[~prefilled].max() <= 1e-3, np.flatnonzero(~prefilled)[err[~prefilled].argmax()]
    assert err[prefilled].max() <= 5e-3, np.flatnonzero(prefilled)[err[prefilled].argmax()]
    for name, got, ref in (("K", kc, k16), ("V", vc, v16)):
        g = O.f16_to_f32(to_host(got).reshape(2, MAX_CTX, 256)[:, :total]).astype(np.float64)
        r = O.f16_to_f32(ref[:, :total]).astype(np.float64)
        # One f16 ulp of the value (the two sides round f32 values that differ by accumulation
        # order) plus 1e-4 of the row's largest magnitude (small rotated entries).
        ulp = np.spacing(np.abs(r).astype(np.float16)).astype(np.float64)
        scale = np.abs(r).max(axis=2, keepdims=True)
        excess = np.abs(g - r) / (ulp + 1e-4 * scale)
        print(f"[layer] {name} cache: {int((g != r).sum())} of {g.size} entries differ, worst "
              f"{excess.max():.2f} of the bound", flush=True)
        assert excess.max() <= 1.0, name


def test_layer_rejections(attn, torch_mod, layer_case):
    torch = torch_mod
    layer, _, _ = layer_case
    kc = torch.zeros(2 * 8 * 256, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    h = torch.zeros(20 * 2048, device="cuda")
    y = torch.zeros_like(h)
    ws = attn.LayerWorkspace(max_tok=16)
    with pytest.raises(RuntimeError, match="KV cache is full"):
        attn.layer_decode(layer, kc, vc, 8, 8, h[:2048], None, y[:2048], EPS, ws)
    with pytest.raises(RuntimeError, match="KV cache is full"):
        attn.layer_prefill(layer, kc, vc, 8, 4, 5, h, None, y, EPS, ws)
    with pytest.raises(RuntimeError, match="does not fit"):
        big_kc = torch.zeros(2 * 64 * 256, dtype=torch.float16, device="cuda")
        attn.layer_prefill(layer, big_kc, torch.zeros_like(big_kc), 64, 0, 17,
                           torch.zeros(17 * 2048, device="cuda"), None,
                           torch.zeros(17 * 2048, device="cuda"), EPS, ws)


def test_layer_prefill_balanced_chunk(O, attn, torch_mod, layer_case):
    """One 512-token chunk on an empty cache: the layer's prefill takes the balanced form with
    split token blocks (chunks of up to 2048 tokens), against the layer oracle."""
    torch = torch_mod
    layer, deq, norms = layer_case
    n = ctx = 512
    rng = np.random.default_rng(512)
    h0 = rng.standard_normal((n, 2048)).astype(np.float32)
    delta = (0.5 * rng.standard_normal((n, 2048))).astype(np.float32)
    h, d = to_dev(torch, h0.reshape(-1)), to_dev(torch, delta.reshape(-1))
    y = torch.full((n * 2048,), -1234.5, dtype=torch.float32, device="cuda")
    kc = torch.zeros(2 * ctx * 256, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    ws = attn.LayerWorkspace(max_tok=n)
    attn.layer_prefill(layer, kc, vc, ctx, 0, n, h, d, y, EPS, ws)
    first = to_host(y).copy()
    h2 = to_dev(torch, h0.reshape(-1))  # the same chunk again over the same workspace
    attn.layer_prefill(layer, kc, vc, ctx, 0, n, h2, d, y, EPS, ws)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(y), first), "repeat over one workspace"
    _, ref_y, _, _ = O.layer_f64(h0, delta, deq["q"], deq["k"], deq["v"], deq["o"],
                                 norms["attn_norm"], norms["q_norm"], norms["k_norm"],
                                 norms["inv_freq"], 0, ctx, EPS)
    got = first.reshape(n, 2048).astype(np.float64)
    err = np.sqrt(((got - ref_y) ** 2).sum(axis=1) / (ref_y ** 2).sum(axis=1))
    print(f"[layer] 512-token balanced chunk: max rel-L2 {err.max():.2e}", flush=True)
    assert np.isfinite(got).all()
    assert err.max() <= 5e-3, int(err.argmax())


def test_layer_core_after_each_call(O, attn, torch_mod, layer_case):
    """The attention output each step leaves in its workspace (the engine's scratch.core after
    attention_decode and ps.core after attention_prefill, which tests/test_attention.hip:68,104
    read) against the layer oracle's core, read after every call: a 13-token prefill, three
    decode steps, a 20-token ingest in chunks of 16 (ps.core holds the last chunk's 4 rows) and a
    decode step. Gates: the reference's own 1e-3 relative L2 per token for decode steps
    (tests/test_attention.hip:71) and 5e-3 for prefill rows (f16 MFMA operands)."""
    torch = torch_mod
    layer, deq, norms = layer_case
    rng = np.random.default_rng(68)
    total = 13 + 3 + 20 + 1
    h0 = rng.standard_normal((total, 2048)).astype(np.float32)
    h = to_dev(torch, h0.reshape(-1))
    y = torch.zeros(total * 2048, dtype=torch.float32, device="cuda")
    kc = torch.zeros(2 * MAX_CTX * 256, dtype=torch.float16, device="cuda")
    vc = torch.zeros_like(kc)
    ws = attn.LayerWorkspace(max_tok=16)
    _, _, _, _, ref_core = O.layer_f64(h0, None, deq["q"], deq["k"], deq["v"], deq["o"],
                                       norms["attn_norm"], norms["q_norm"], norms["k_norm"],
                                       norms["inv_freq"], 0, MAX_CTX, EPS, with_core=True)

    def rows(t, a, b):
        return t[a * 2048:b * 2048]

    def check(got, a, b, gate, what):
        got = to_host(got).reshape(b - a, 4096).astype(np.float64)
        ref = ref_core[a:b]
        err = np.sqrt(((got - ref) ** 2).sum(axis=1) / (ref ** 2).sum(axis=1))
        print(f"[layer core] {what} tokens {a}..{b - 1}: max rel-L2 {err.max():.2e}", flush=True)
        assert np.isfinite(got).all() and err.max() <= gate, (what, a + int(err.argmax()))

    attn.layer_prefill(layer, kc, vc, MAX_CTX, 0, 13, rows(h, 0, 13), None, rows(y, 0, 13), EPS,
                       ws)
    torch.cuda.synchronize()
    check(ws.prefill_core[:13], 0, 13, 5e-3, "prefill")
    for t in range(13, 16):
        attn.layer_decode(layer, kc, vc, MAX_CTX, t, rows(h, t, t + 1), None, rows(y, t, t + 1),
                          EPS, ws)
        torch.cuda.synchronize()
        check(ws.decode_core, t, t + 1, 1e-3, "decode")
    attn.layer_ingest(layer, kc, vc, MAX_CTX, 16, 20, rows(h, 16, 36), None, rows(y, 16, 36), EPS,
                      ws, chunk=16)
    torch.cuda.synchronize()
    check(ws.prefill_core[:4], 32, 36, 5e-3, "ingest's last chunk")
    attn.layer_decode(layer, kc, vc, MAX_CTX, 36, rows(h, 36, 37), None, rows(y, 36, 37), EPS, ws)
    torch.cuda.synchronize()
    check(ws.decode_core, 36, 37, 1e-3, "decode")
