"""fp8 (e4m3 rows) KV cache on MI355X, through the C ABI, against the oracle.

  * encode: codes and scales bit-identical to the oracle's nearest-code encoder;
  * decode: split + combine over e4m3 rows against oracle_decode_fp8_f64 on the same codes and
    scales, gate |got - ref| <= 2e-3 + 1e-2 |ref| and, since the split computes at the f16
    path's precision (f32 query and numerators as f16 pairs, f32 sums), the reference's per-head
    rel-L2 <= 1e-5; over the reference's boundary lengths, the C2 size, every code value, and
    with NaN codes past len (a read past the cache would show);
  * prep: the q output bit-identical to attn_prep's, V codes bit-identical to the oracle's, K
    within half a code step of the oracle's normalised, rotated row;
  * the format's own error against the f16 cache (reported, bounded loosely): it is a property
    of e4m3 storage, not of the kernels;
  * prefill over e4m3 rows: the f16 workspace rows bit-identical to f16(scale e4m3(code)) with
    saturation at 65504, the prefill against the FP64 prefill oracle over those rows (same
    gate), and the batched e4m3 prep bit-identical to the single-token one.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REF_REL_L2, report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, KV, D = 16, 2, 256
CANARY = -9123.5


def encode_host(O, k16, v16, max_ctx):
    kf = O.f16_to_f32(k16).reshape(KV * max_ctx, D)
    vf = O.f16_to_f32(v16).reshape(KV * max_ctx, D)
    return O.fp8_encode_rows(kf) + O.fp8_encode_rows(vf)  # k8, ks, v8, vs


def upload(attn, torch, k8, ks, v8, vs, max_ctx):
    c = attn.Fp8Cache(max_ctx)
    c.k8.copy_(torch.from_numpy(k8.reshape(-1)))
    c.v8.copy_(torch.from_numpy(v8.reshape(-1)))
    c.k_scale.copy_(torch.from_numpy(ks.reshape(-1)))
    c.v_scale.copy_(torch.from_numpy(vs.reshape(-1)))
    return c


def run_decode_fp8(attn, torch, q, qg, cache, length, max_splits, n_splits=None):
    core = torch.full((H * D,), CANARY, dtype=torch.float32, device="cuda")
    sc = attn.DecodeScratch(max_splits)
    n = attn.attn_decode_fp8(to_dev(torch, q), to_dev(torch, qg), cache, core, sc, length,
                             n_splits)
    torch.cuda.synchronize()
    out = to_host(core).reshape(H, D)
    assert not (out == CANARY).any(), "unwritten outputs"
    return out, n


def test_encode_kernel_bit_identical(O, attn, torch_mod):
    torch = torch_mod
    max_ctx, pos0, n = 300, 37, 250
    d = O.decode_inputs(41, max_ctx, max_ctx)
    k16 = d["k"].reshape(KV, max_ctx, D).copy()
    v16 = d["v"].reshape(KV, max_ctx, D).copy()
    k16[0, 40] = 0                                       # zero row
    k16[1, 41] = O.f32_to_f16(np.full(D, 6e-8, np.float32))   # f16 subnormals
    v16[0, 42] = O.f32_to_f16(np.linspace(-65504, 65504, D).astype(np.float32))  # f16 extremes
    mids = (O.e4m3_table()[0x38:0x40] + O.e4m3_table()[0x39:0x41]) / 2  # exact ties at scale 1
    v16[1, 43] = O.f32_to_f16(np.resize(mids * (2.0 ** -7) * 128, D).astype(np.float32))
    kc, vc = to_dev(torch, k16.reshape(-1)), to_dev(torch, v16.reshape(-1))
    cache = attn.Fp8Cache(max_ctx)
    cache.k8.fill_(0xAB)
    cache.k_scale.fill_(-1.0)
    attn.attn_kv_encode_fp8(kc, vc, cache, pos0, n)
    torch.cuda.synchronize()
    k8, ks, v8, vs = encode_host(O, k16.reshape(-1), v16.reshape(-1), max_ctx)
    rows = np.zeros((KV, max_ctx), bool)
    rows[:, pos0:pos0 + n] = True
    rows = rows.reshape(-1)
    gk8 = to_host(cache.k8).reshape(KV * max_ctx, D)
    gks = to_host(cache.k_scale)
    assert np.array_equal(gk8[rows], k8[rows]) and np.array_equal(gks[rows], ks[rows])
    assert np.array_equal(to_host(cache.v8).reshape(-1, D)[rows], v8[rows])
    assert np.array_equal(to_host(cache.v_scale)[rows], vs[rows])
    assert (gk8[~rows] == 0xAB).all() and (gks[~rows] == -1.0).all()  # nothing else written


@pytest.mark.parametrize("length", [1, 15, 16, 17, 63, 64, 65, 257, 1000, 4101])
def test_decode_fp8_boundaries(O, attn, torch_mod, length):
    torch = torch_mod
    max_ctx = length + 21
    d = O.decode_inputs(length, length, max_ctx, q_scale=2.0)
    k8, ks, v8, vs = encode_host(O, d["k"], d["v"], max_ctx)
    # rows past len hold NaN codes and NaN scales: any read of them would poison the output
    for a in (k8, v8):
        a.reshape(KV, max_ctx, D)[:, length:] = 0x7F
    for a in (ks, vs):
        a.reshape(KV, max_ctx)[:, length:] = np.nan
    cache = upload(attn, torch, k8, ks, v8, vs, max_ctx)
    ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs, length, max_ctx)
    for cap in (60, 128):
        got, n = run_decode_fp8(attn, torch, d["q"], d["qg"], cache, length, cap)
        st = O.compare(got, ref)
        report(f"fp8 decode len={length} splits={n}", st)
        assert st["ok"] and st["rel_l2_head"] <= REF_REL_L2, st


def test_decode_fp8_c2_and_format_error(O, attn, torch_mod):
    """C2 (32768 keys, q/K/V N(0,1) from seed = len): parity with the oracle on the e4m3 rows,
    independence of the split count, and the format's error against the f16 cache."""
    torch = torch_mod
    L = 32768
    d = O.decode_inputs(L, L, L, q_scale=1.0)
    k8, ks, v8, vs = encode_host(O, d["k"], d["v"], L)
    cache = upload(attn, torch, k8, ks, v8, vs, L)
    ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs, L, L)
    outs = []
    for n in (128, 1, 7):
        got, _ = run_decode_fp8(attn, torch, d["q"], d["qg"], cache, L, 128, n)
        st = O.compare(got, ref)
        report(f"fp8 decode C2 splits={n}", st)
        assert st["ok"] and st["rel_l2_head"] <= REF_REL_L2, st
        outs.append(got)
    for o in outs[1:]:
        assert O.compare(o, outs[0].astype(np.float64))["ok"]
    ref16 = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], L, L)
    st = O.compare(outs[0], ref16)
    report("fp8 format vs f16 cache, C2", st)
    assert st["rel_l2"] < 0.05, st


def test_decode_fp8_every_code(O, attn, torch_mod):
    """Random bytes over every finite code (both signs, subnormals, 448) with random
    power-of-two row scales: each code's widening to f16 and both scale paths are exercised."""
    torch = torch_mod
    L = max_ctx = 2048
    rng = np.random.default_rng(17)
    finite = np.array([c for c in range(256) if c & 0x7F != 0x7F], np.uint8)
    k8 = rng.choice(finite, size=(KV * L, D)).astype(np.uint8)
    v8 = rng.choice(finite, size=(KV * L, D)).astype(np.uint8)
    ks = (2.0 ** rng.integers(-11, -8, KV * L)).astype(np.float32)
    vs = (2.0 ** rng.integers(-9, -3, KV * L)).astype(np.float32)
    d = O.decode_inputs(3, L, L, q_scale=1.0)
    cache = upload(attn, torch, k8, ks, v8, vs, max_ctx)
    ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs, L, max_ctx)
    got, n = run_decode_fp8(attn, torch, d["q"], d["qg"], cache, L, 128)
    st = O.compare(got, ref)
    report(f"fp8 decode every code splits={n}", st)
    assert st["ok"] and st["rel_l2_head"] <= REF_REL_L2, st


def test_decode_fp8_v_scale_range(O, attn, torch_mod):
    """The V row scales enter the numerators only relative to a reference scale (the largest of
    the tiles a wave has met, a power of two), and O is multiplied by that reference in f32. So
    multiplying every V scale by 2^k (V rows near 2^-12 .. 2^-20 for k = -14, max |v| near 2^15
    for k = 13) multiplies the output by exactly 2^k, bit for bit, as the exact result does; and
    rows whose scales spread over 2^8 (2^-12 .. 2^-20) stay within a relative tolerance of the
    oracle."""
    torch = torch_mod
    L = max_ctx = 4101
    d = O.decode_inputs(L, L, max_ctx, q_scale=2.0)
    k8, ks, v8, vs = encode_host(O, d["k"], d["v"], max_ctx)
    base = None
    for k in (0, -14, 13):
        cache = upload(attn, torch, k8, ks, v8, (vs * np.float32(2.0 ** k)).astype(np.float32),
                       max_ctx)
        got, _ = run_decode_fp8(attn, torch, d["q"], d["qg"], cache, L, 128)
        if base is None:
            base = got
            ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs, L, max_ctx)
            st = O.compare(got, ref)
            report("fp8 decode unscaled", st)
            assert st["ok"], st
        else:
            assert np.isfinite(got).all()
            assert np.array_equal(got, (base.astype(np.float64) * 2.0 ** k).astype(np.float32)), k
    rng = np.random.default_rng(23)
    vs_mixed = (vs * 2.0 ** (-12 - rng.integers(0, 9, vs.size))).astype(np.float32)
    cache = upload(attn, torch, k8, ks, v8, vs_mixed, max_ctx)
    got, n = run_decode_fp8(attn, torch, d["q"], d["qg"], cache, L, 128)
    ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs_mixed, L, max_ctx)
    st = O.compare(got, ref)
    report(f"fp8 decode V scales 2^-12..2^-20 splits={n}", st)
    assert np.isfinite(got).all() and st["rel_l2_head"] < 2e-3, st


def test_prep_fp8_and_engine_sequence(O, attn, torch_mod):
    """prep_fp8 at several positions: q equals attn_prep's bit for bit, V codes equal the
    oracle's, K within half a code step of the oracle's row; then decode over the cache the
    appends built, against the oracle on the same codes."""
    torch = torch_mod
    PROJ, EPS = 9216, 1e-6
    rng = np.random.default_rng(77)
    q_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    k_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    inv = O.inv_freq(10_000_000.0)
    w = [to_dev(torch, a) for a in (q_norm, k_norm, inv)]
    max_ctx, P = 700, 640
    d = O.decode_inputs(7, P, max_ctx)
    k8, ks, v8, vs = encode_host(O, d["k"], d["v"], max_ctx)
    cache = upload(attn, torch, k8, ks, v8, vs, max_ctx)  # positions >= P are overwritten below
    kc16 = torch.zeros(KV * max_ctx * D, dtype=torch.float16, device="cuda")
    vc16 = torch.zeros_like(kc16)
    q8 = torch.empty(H * D, device="cuda")
    q16 = torch.empty(H * D, device="cuda")
    out = torch.empty(H * D, device="cuda")
    sc = attn.DecodeScratch(128)
    for i in range(12):
        pos = P + i
        proj = O.normal(900 + pos, PROJ)
        dp = to_dev(torch, proj)
        attn.attn_prep_fp8(dp[:8192], dp[8192:8704], dp[8704:], *w, cache, q8, pos, EPS)
        attn.attn_prep(dp[:8192], dp[8192:8704], dp[8704:], *w, kc16, vc16, q16, pos, max_ctx,
                       EPS)
        attn.attn_decode_fp8(q8, dp[:8192], cache, out, sc, pos + 1)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(q8), to_host(q16))
        _, k_ref, _ = O.prep_f64(proj[:8192], proj[8192:8704], proj[8704:], q_norm, k_norm, inv,
                                 pos, EPS)
        g8 = to_host(cache.k8).reshape(KV, max_ctx, D)[:, pos]
        gs = to_host(cache.k_scale).reshape(KV, max_ctx)[:, pos]
        gv8 = to_host(cache.v8).reshape(KV, max_ctx, D)[:, pos]
        gvs = to_host(cache.v_scale).reshape(KV, max_ctx)[:, pos]
        v_codes, v_scales = O.fp8_encode_rows(proj[8704:].reshape(KV, D))
        assert np.array_equal(gv8, v_codes) and np.array_equal(gvs, v_scales)
        kx = O.f16_to_f32(k_ref).astype(np.float64)  # the oracle's row, f16-rounded
        deq = O.fp8_dequant(g8, gs)
        assert np.all(np.abs(deq - kx) <= np.abs(kx) * (2.0 ** -4 + 2.0 ** -10)
                      + gs[:, None] * 2.0 ** -9 + 1e-6)
        kh, vh = to_host(cache.k8), to_host(cache.v8)
        ref = O.decode_fp8_f64(to_host(q8), proj[:8192], kh, vh, to_host(cache.k_scale),
                               to_host(cache.v_scale), pos + 1, max_ctx)
        st = O.compare(to_host(out).reshape(H, D), ref)
        report(f"fp8 engine decode len={pos + 1}", st)
        assert st["ok"], st


def widen_host(O, codes, scales):
    """Rows as attn_prefill_fp8 widens them: f16(clamp(scale * e4m3(code), +-65504)), RNE. The
    product is exact in f32, so the float64 dequant rounded once to f16 is the same value."""
    val = np.clip(O.fp8_dequant(codes, scales), -65504.0, 65504.0).astype(np.float32)
    return O.f32_to_f16(val)


def run_prefill_fp8(attn, torch, p, cache):
    n, S = p["n"], p["qg_stride"]
    core = torch.full((n * H * D,), CANARY, dtype=torch.float32, device="cuda")
    ws = attn.attn_prefill_fp8(to_dev(torch, p["q"]), to_dev(torch, p["qg"]), cache, core,
                               p["pos0"], n, qg_stride=S)
    torch.cuda.synchronize()
    out = to_host(core).reshape(n, H, D)
    assert not (out == CANARY).any(), "unwritten outputs"
    return out, ws


def test_prefill_fp8_widening_bit_exact(O, attn, torch_mod):
    """The f16 workspace rows equal f16(scale * e4m3(code)) for every finite code, scales from
    2^-107 to 2^8, and saturate at 65504 where a code of 256 meets the largest scale."""
    torch = torch_mod
    rows = 300
    max_ctx = rows + 3
    rng = np.random.default_rng(31)
    finite = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], dtype=np.uint8)
    k8 = rng.choice(finite, size=(KV, max_ctx, D)).astype(np.uint8)
    v8 = rng.choice(finite, size=(KV, max_ctx, D)).astype(np.uint8)
    k8[:, :2, :len(finite)] = finite  # every finite code at least once
    ks = (2.0 ** rng.integers(-107, 9, size=(KV, max_ctx))).astype(np.float32)
    vs = (2.0 ** rng.integers(-107, 9, size=(KV, max_ctx))).astype(np.float32)
    ks[:, 5] = vs[:, 5] = 256.0
    k8[:, 5, :4] = v8[:, 5, :4] = [0x78, 0xF8, 0x77, 0x70]  # 256, -256, 240, 128 at scale 2^8
    cache = upload(attn, torch, k8, ks, v8, vs, max_ctx)
    p = O.prefill_inputs(5, rows - 1, 1, max_ctx)
    out, ws = run_prefill_fp8(attn, torch, p, cache)
    assert np.isfinite(out).all()
    gk = to_host(ws.k).view(np.uint16).reshape(KV, rows, D)
    gv = to_host(ws.v).view(np.uint16).reshape(KV, rows, D)
    assert np.array_equal(gk, widen_host(O, k8[:, :rows], ks[:, :rows]))
    assert np.array_equal(gv, widen_host(O, v8[:, :rows], vs[:, :rows]))
    assert O.f16_to_f32(gk[:, 5, :2]).tolist() == [[65504.0, -65504.0]] * KV


@pytest.mark.parametrize("pos0,n", [(0, 1), (0, 33), (40, 17), (100, 128), (1000, 77)])
def test_prefill_fp8_matches_oracle(O, attn, torch_mod, pos0, n):
    """Prefill over e4m3 rows against the FP64 prefill oracle over the same rows widened to f16
    (the kernel's f16 operands), every row, gate |got - ref| <= 2e-3 + 1e-2 |ref|."""
    torch = torch_mod
    max_ctx = pos0 + n + 5
    p = O.prefill_inputs(3000 + pos0 + n, pos0, n, max_ctx, q_scale=2.0)
    k8, ks, v8, vs = encode_host(O, p["k"], p["v"], max_ctx)
    cache = upload(attn, torch, k8, ks, v8, vs, max_ctx)
    got, _ = run_prefill_fp8(attn, torch, p, cache)
    kw = widen_host(O, k8, ks).reshape(-1)
    vw = widen_host(O, v8, vs).reshape(-1)
    ref = O.prefill_f64(p["q"], p["qg"], p["qg_stride"], kw, vw, pos0, max_ctx, np.arange(n))
    st = O.compare(got, ref)
    report(f"fp8 prefill pos0={pos0} n={n}", st)
    assert st["ok"], st


def test_prep_batch_fp8_equals_single_token_prep(O, attn, torch_mod):
    """prep_batch_fp8 over 37 tokens writes the same e4m3 rows, scales and q as 37 calls of
    prep_fp8, bit for bit."""
    torch = torch_mod
    PROJ, EPS, n, pos0, max_ctx = 9216, 1e-6, 37, 5, 64
    rng = np.random.default_rng(41)
    q_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    k_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    w = [to_dev(torch, a) for a in (q_norm, k_norm, O.inv_freq(10_000_000.0))]
    proj = to_dev(torch, O.normal(4242, n * PROJ))
    a, b = attn.Fp8Cache(max_ctx), attn.Fp8Cache(max_ctx)
    qa = torch.empty(n * H * D, device="cuda")
    qb = torch.empty(n * H * D, device="cuda")
    attn.attn_prep_batch_fp8(proj, proj[8192:], proj[8704:], *w, a, qa, pos0, n, PROJ, EPS)
    for t in range(n):
        r = proj[t * PROJ:(t + 1) * PROJ]
        attn.attn_prep_fp8(r[:8192], r[8192:8704], r[8704:], *w, b, qb[t * H * D:(t + 1) * H * D],
                           pos0 + t, EPS)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(qa), to_host(qb))
    for x, y in zip(a.buffers(), b.buffers()):
        assert np.array_equal(to_host(x), to_host(y))


def test_prep_batch_fp8_then_prefill_fp8(O, attn, torch_mod):
    """The engine's prefill over an e4m3 cache: a 300-token prompt prepped in one batch, then
    the prefill over the cache it built, against the oracle over the widened rows."""
    torch = torch_mod
    PROJ, EPS, n, max_ctx = 9216, 1e-6, 300, 320
    rng = np.random.default_rng(43)
    q_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    k_norm = (1 + 0.1 * rng.standard_normal(D)).astype(np.float32)
    w = [to_dev(torch, a) for a in (q_norm, k_norm, O.inv_freq(10_000_000.0))]
    proj_h = O.normal(4343, n * PROJ)
    proj = to_dev(torch, proj_h)
    cache = attn.Fp8Cache(max_ctx)
    q = torch.empty(n * H * D, device="cuda")
    attn.attn_prep_batch_fp8(proj, proj[8192:], proj[8704:], *w, cache, q, 0, n, PROJ, EPS)
    core = torch.full((n * H * D,), CANARY, dtype=torch.float32, device="cuda")
    attn.attn_prefill_fp8(q, proj, cache, core, 0, n, qg_stride=PROJ)
    torch.cuda.synchronize()
    got = to_host(core).reshape(n, H, D)
    kw = widen_host(O, to_host(cache.k8).reshape(KV, max_ctx, D),
                    to_host(cache.k_scale).reshape(KV, max_ctx)).reshape(-1)
    vw = widen_host(O, to_host(cache.v8).reshape(KV, max_ctx, D),
                    to_host(cache.v_scale).reshape(KV, max_ctx)).reshape(-1)
    ref = O.prefill_f64(to_host(q), proj_h, PROJ, kw, vw, 0, max_ctx, np.arange(n))
    st = O.compare(got, ref)
    report(f"fp8 prep_batch + prefill n={n}", st)
    assert st["ok"], st
