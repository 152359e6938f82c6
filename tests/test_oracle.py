"""CPU tests pinning the oracle (oracle/attn_oracle.c) before it is trusted as the checker.

Pins, per oracle function:
  generator        published splitmix64 / xoshiro256** known answers; binary16 rounding vs numpy
                   (an independent implementation) over every half pattern and 5M floats.
  decode/prefill   torch float64 scaled_dot_product_attention fixtures (tests/golden); closed forms
                   (one key, constant values, zero query, one dominant key); key-permutation
                   invariance; a GQA grouping check; the causal offset via prefill row == decode.
  partials         LSE-merging the partials of any split equals the full decode; empty span.
  combine (f32)    equals the float64 LSE merge within f32 rounding; empty splits drop out.
  prep             RMSNorm closed form, rotation norm preservation, pos 0 identity, a
                   hand-computed rotation, inv_freq against its formula.
  ref n_splits     the values asserted by the reference's own test
                   (tests/test_attn_splitk.hip:286-290).
"""
from __future__ import annotations

import hashlib
from pathlib import Path

import numpy as np
import pytest

H, KV, D = 16, 2, 256
GOLDEN = Path(__file__).resolve().parent / "golden" / "sdpa_cases.npz"


def sig(x):
    return 1.0 / (1.0 + np.exp(-x.astype(np.float64)))


# ---------------------------------------------------------------------------- generator

def test_splitmix64_known_answers(O):
    assert [int(x) for x in O.splitmix64_stream(0, 3)] == [
        0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [int(x) for x in O.splitmix64_stream(1234567, 2)] == [
        6457827717110365317, 3203168211198807973]


def test_xoshiro256ss_known_answers(O):
    assert [int(x) for x in O.xoshiro_raw([1, 2, 3, 4], 4)] == [
        11520, 0, 1509978240, 1215971899390074240]


def test_f16_round_to_nearest_even_matches_numpy(O):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(1_000_000).astype(np.float32) * s
                        for s in (1e-8, 1e-5, 1.0, 100.0, 6e4)])
    edge = np.array([0.0, -0.0, np.inf, -np.inf, 65504, 65519.99, 65520, 2.0**-24, 2.0**-25,
                     3 * 2.0**-26, 2.0**-14, 1.5 * 2.0**-15, 1 + 2.0**-11, 1 + 3 * 2.0**-11],
                    np.float32)
    x = np.concatenate([x, edge, -edge])
    with np.errstate(over="ignore"):
        expect = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(x), expect)
    bits = np.arange(65536, dtype=np.uint16)
    back, want = O.f16_to_f32(bits), bits.view(np.float16).astype(np.float32)
    same = (back == want) | (np.isnan(back) & np.isnan(want))
    assert same.all()


def test_normal_stream_statistics(O):
    z = O.normal(11, 2_000_000).astype(np.float64)
    assert abs(z.mean()) < 3e-3 and abs(z.var() - 1) < 5e-3
    assert abs(np.mean(z ** 4) - 3) < 3e-2  # Gaussian kurtosis


# ---------------------------------------------------------------------------- golden fixtures

def _digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return np.frombuffer(h.digest(), dtype=np.uint8)


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_generator_matches_fixture(O, golden):
    assert np.array_equal(O.normal(7, 16), golden["gen_normal_seed7"])
    assert np.array_equal(O.normal_f16(7, 16), golden["gen_normal_f16_seed7"])


@pytest.mark.parametrize("length", [1, 7, 33])
def test_decode_oracle_matches_torch_sdpa(O, golden, length):
    seed, n, max_ctx, scale = (int(x) for x in golden[f"decode_{length}_meta"])
    d = O.decode_inputs(seed, n, max_ctx, q_scale=float(scale))
    assert np.array_equal(_digest(d["q"], d["qg"], d["k"], d["v"]),
                          golden[f"decode_{length}_sha256"])
    got = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], n, max_ctx)
    np.testing.assert_allclose(got, golden[f"decode_{length}_out"], rtol=1e-11, atol=1e-13)


@pytest.mark.parametrize("case", ["0_5", "9_4", "31_3"])
def test_prefill_oracle_matches_torch_sdpa(O, golden, case):
    seed, pos0, n, max_ctx = (int(x) for x in golden[f"prefill_{case}_meta"])
    p = O.prefill_inputs(seed, pos0, n, max_ctx, q_scale=2.0)
    assert np.array_equal(_digest(p["q"], p["qg"], p["k"], p["v"]),
                          golden[f"prefill_{case}_sha256"])
    got = O.prefill_f64(p["q"], p["qg"], p["qg_stride"], p["k"], p["v"], pos0, max_ctx,
                        np.arange(n))
    np.testing.assert_allclose(got, golden[f"prefill_{case}_out"], rtol=1e-11, atol=1e-13)


# ---------------------------------------------------------------------------- closed forms

def _decode_case(O, length, max_ctx=None, seed=3):
    return O.decode_inputs(seed, length, max_ctx or length + 1, q_scale=2.0)


def test_decode_single_key_is_value_times_gate(O):
    d = _decode_case(O, 1, 4)
    out = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], 1, 4)
    v = O.f16_to_f32(d["v"]).reshape(KV, 4, D)[:, 0].astype(np.float64)
    g = sig(d["qg"].reshape(H, 2 * D)[:, D:])
    expect = np.repeat(v, 8, axis=0) * g
    np.testing.assert_allclose(out, expect, rtol=1e-14, atol=0)


def test_decode_constant_values_and_zero_query(O):
    L, M = 50, 51
    d = _decode_case(O, L, M)
    qg = d["qg"]
    g = sig(qg.reshape(H, 2 * D)[:, D:])
    # constant V rows: every head returns c * sigmoid(gate) regardless of q
    vc = np.tile(O.f32_to_f16(np.linspace(-2, 2, D).astype(np.float32)), KV * M)
    out = O.decode_f64(d["q"], qg, d["k"], vc, L, M)
    c = O.f16_to_f32(vc[:D]).astype(np.float64)
    np.testing.assert_allclose(out, c[None, :] * g, rtol=1e-13, atol=1e-15)
    # zero query: uniform softmax -> mean of the visible V rows of the head's group
    out = O.decode_f64(np.zeros(H * D, np.float32), qg, d["k"], d["v"], L, M)
    v = O.f16_to_f32(d["v"]).reshape(KV, M, D)[:, :L].astype(np.float64)
    np.testing.assert_allclose(out, np.repeat(v.mean(axis=1), 8, axis=0) * g, rtol=1e-12,
                               atol=1e-15)


def test_decode_dominant_key_and_gqa_grouping(O):
    L, M = 40, 40
    d = _decode_case(O, L, M)
    k = O.f16_to_f32(d["k"]).reshape(KV, M, D)
    v = O.f16_to_f32(d["v"]).reshape(KV, M, D).astype(np.float64)
    # query of head h = 40 * K[kvh(h)][j_h]: softmax collapses onto key j_h of ITS kv head
    js = [(5 * h + 3) % L for h in range(H)]
    q = np.stack([40.0 * k[h // 8, js[h]] for h in range(H)]).astype(np.float32).ravel()
    out = O.decode_f64(q, d["qg"], d["k"], d["v"], L, M)
    g = sig(d["qg"].reshape(H, 2 * D)[:, D:])
    expect = np.stack([v[h // 8, js[h]] for h in range(H)]) * g
    np.testing.assert_allclose(out, expect, rtol=1e-6, atol=1e-6)


def test_decode_key_permutation_invariance(O):
    L, M = 64, 64
    d = _decode_case(O, L, M)
    perm = np.random.default_rng(1).permutation(L)
    k = d["k"].reshape(KV, M, D)[:, perm].ravel()
    v = d["v"].reshape(KV, M, D)[:, perm].ravel()
    a = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], L, M)
    b = O.decode_f64(d["q"], d["qg"], k, v, L, M)
    np.testing.assert_allclose(a, b, rtol=1e-12, atol=1e-15)


def test_prefill_row_equals_decode_at_its_length(O):
    pos0, n = 21, 6
    p = O.prefill_inputs(17, pos0, n, pos0 + n, q_scale=2.0)
    rows = O.prefill_f64(p["q"], p["qg"], p["qg_stride"], p["k"], p["v"], pos0, p["max_ctx"],
                         np.arange(n))
    for t in range(n):
        qg_t = p["qg"][t * p["qg_stride"]: t * p["qg_stride"] + H * 2 * D]
        dec = O.decode_f64(p["q"][t * H * D:(t + 1) * H * D], qg_t, p["k"], p["v"],
                           pos0 + t + 1, p["max_ctx"])
        np.testing.assert_array_equal(rows[t], dec)
    # one key fewer must differ (the causal limit is inclusive of position pos0 + t)
    dec_short = O.decode_f64(p["q"][:H * D], p["qg"][:H * 2 * D], p["k"], p["v"], pos0,
                             p["max_ctx"])
    assert np.abs(dec_short - rows[0]).max() > 1e-6


def test_partials_merge_to_decode(O):
    L, M = 300, 310
    d = _decode_case(O, L, M)
    full = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], L, M)
    cuts = [0, 1, 64, 65, 200, 300]
    g = sig(d["qg"].reshape(H, 2 * D)[:, D:])
    for kvh in range(KV):
        parts = [O.partials_f64(d["q"], d["k"], d["v"], kvh, M, a, b)
                 for a, b in zip(cuts[:-1], cuts[1:])]
        ms = np.stack([p[0] for p in parts])
        Mx = ms.max(axis=0)
        w = np.exp(ms - Mx)
        l = (w * np.stack([p[1] for p in parts])).sum(axis=0)
        o = (w[:, :, None] * np.stack([p[2] for p in parts])).sum(axis=0)
        merged = o / l[:, None] * g[8 * kvh: 8 * kvh + 8]
        np.testing.assert_allclose(merged, full[8 * kvh: 8 * kvh + 8], rtol=1e-12, atol=1e-15)
    m, l, o = O.partials_f64(d["q"], d["k"], d["v"], 0, M, 7, 7)
    assert np.all(np.isneginf(m)) and not l.any() and not o.any()


def test_combine_f32_matches_float64_merge(O):
    rng = np.random.default_rng(5)
    for n_splits in (1, 3, 60, 129):
        pm = rng.uniform(-3, 3, (KV, n_splits, 8)).astype(np.float32)
        pm[:, 1::3] += 80
        pl = (1 + np.abs(rng.uniform(-3, 3, pm.shape))).astype(np.float32)
        po = rng.uniform(-3, 3, pm.shape + (D,)).astype(np.float32)
        if n_splits > 2:  # empty splits: (-inf, 0, 0)
            pm[:, 2], pl[:, 2], po[:, 2] = -np.inf, 0, 0
        qg = rng.uniform(-3, 3, H * 2 * D).astype(np.float32)
        got = O.combine_f32(pm, pl, po, qg, n_splits)
        m64 = pm.astype(np.float64)
        w = np.exp(m64 - m64.max(axis=1, keepdims=True))
        L = (w * pl).sum(axis=1)
        o = (w[..., None] * po).sum(axis=1) / L[..., None]
        expect = o.reshape(H, D) * sig(qg.reshape(H, 2 * D)[:, D:])
        np.testing.assert_allclose(got, expect, rtol=2e-5, atol=1e-6)


# ---------------------------------------------------------------------------- prep

def test_prep_closed_forms(O):
    rng = np.random.default_rng(9)
    qg = rng.standard_normal(H * 2 * D).astype(np.float32)
    k = rng.standard_normal(KV * D).astype(np.float32)
    v = rng.standard_normal(KV * D).astype(np.float32)
    ones = np.ones(D, np.float32)
    inv = O.inv_freq(10_000_000.0)
    expect_inv = (1.0 / np.power(np.float32(10_000_000.0),
                                 np.arange(0, 64, 2, dtype=np.float32) / np.float32(64)))
    np.testing.assert_allclose(inv, expect_inv.astype(np.float32), rtol=2e-7)
    eps = 1e-6
    # pos 0: no rotation; with unit weights every head has rms 1 / sqrt(1 + eps / ms)
    q0, k0, v0 = O.prep_f64(qg, k, v, ones, ones, inv, 0, eps)
    x = qg.reshape(H, 2 * D)[:, :D].astype(np.float64)
    ms = (x ** 2).mean(axis=1, keepdims=True)
    np.testing.assert_allclose(q0, x / np.sqrt(ms + eps), rtol=1e-12)
    assert np.array_equal(v0, O.f32_to_f16(v.reshape(KV, D)))
    kx = k.reshape(KV, D).astype(np.float64)
    kn = kx / np.sqrt((kx ** 2).mean(axis=1, keepdims=True) + eps)
    assert np.array_equal(k0, O.f32_to_f16(kn.astype(np.float32)))
    # pos 7: pairs (i, i + 32), i < 32, rotate by 7 * inv_freq[i]; dims >= 64 untouched
    q7, _, _ = O.prep_f64(qg, k, v, ones, ones, inv, 7, eps)
    y = x / np.sqrt(ms + eps)
    th = (np.float32(7) * inv).astype(np.float64)
    np.testing.assert_allclose(q7[:, :32], y[:, :32] * np.cos(th) - y[:, 32:64] * np.sin(th),
                               rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(q7[:, 32:64], y[:, 32:64] * np.cos(th) + y[:, :32] * np.sin(th),
                               rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(q7[:, 64:], y[:, 64:], rtol=1e-13)
    np.testing.assert_allclose(q7[:, :32] ** 2 + q7[:, 32:64] ** 2,
                               y[:, :32] ** 2 + y[:, 32:64] ** 2, rtol=1e-12)
    # weights scale dims
    w = np.linspace(0.5, 1.5, D).astype(np.float32)
    qw, _, _ = O.prep_f64(qg, k, v, w, ones, inv, 0, eps)
    np.testing.assert_allclose(qw, q0 * w, rtol=1e-12)


# ---------------------------------------------------------------------------- policy

def test_reference_split_policy_values(O):
    # tests/test_attn_splitk.hip:286-290 asserts these for the reference's attn_n_splits.
    assert O.ref_n_splits(3872, 60) == 21
    assert O.ref_n_splits(33, 60) == 2
    assert O.ref_n_splits(4096, 60) == 22
    assert O.ref_n_splits(16384, 60) == 57
    assert O.ref_n_splits(288, 60) == 9
    assert O.ref_n_splits(0, 60) == 1
    assert O.ref_n_splits(32768, 60) == 57  # the 32k row of the survey


def test_ragged_oracle_equals_decode_per_sequence(O):
    lens = np.array([1, 5, 40, 17], np.uint32)
    r = O.ragged_inputs(4, lens)
    out = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    for s, L in enumerate(lens):
        L = int(L)
        off = int(r["offsets"][s])
        k = r["k"][off: off + KV * L * D]
        v = r["v"][off: off + KV * L * D]
        qg = np.zeros((H, 2 * D), np.float32)
        qg[:, D:] = r["gate"][s * H * D:(s + 1) * H * D].reshape(H, D)
        dec = O.decode_f64(r["q"][s * H * D:(s + 1) * H * D], qg.ravel(), k, v, L, L)
        np.testing.assert_array_equal(out[s], dec)


def test_layer_oracle_single_token_closed_form():
    """At position 0 the attention sees one key: softmax = 1, so head h's core is the f16 V row
    of its KV head times sigmoid(gate), and y = W_o f16(core) -- independent of decode_f64. The
    residual update and the cache row come out of the same call."""
    from oracle import oracle as O
    rng = np.random.default_rng(5)
    wq = rng.standard_normal((8192, 2048)) * 0.02
    wk = rng.standard_normal((512, 2048)) * 0.02
    wv = rng.standard_normal((512, 2048)) * 0.02
    wo = rng.standard_normal((2048, 4096)) * 0.02
    an, qn, kn = (1 + 0.1 * rng.standard_normal(n) for n in (2048, 256, 256))
    h = rng.standard_normal((1, 2048)).astype(np.float32)
    dl = rng.standard_normal((1, 2048)).astype(np.float32)
    hh, y, k16, v16 = O.layer_f64(h, dl, wq, wk, wv, wo, an, qn, kn, O.inv_freq(1e7), 0, 4, 1e-6)
    assert np.array_equal(hh, (h + dl).astype(np.float32))
    hs = (h + dl).astype(np.float64)
    xn = hs / np.sqrt((hs * hs).mean() + 1e-6) * an   # RMSNorm, restated from its definition
    xn = xn.astype(np.float32).astype(np.float16).astype(np.float64)
    proj = np.concatenate([xn @ w.T for w in (wq, wk, wv)], axis=1).astype(np.float32)[0]
    v_rows = O.f16_to_f32(v16[:, 0]).astype(np.float64)          # [2][256], position 0
    assert np.array_equal(v16[:, 0], O.f32_to_f16(proj[8704:].reshape(2, 256)))
    gate = proj[:8192].reshape(16, 512)[:, 256:].astype(np.float64)
    core = np.stack([v_rows[hd // 8] / (1 + np.exp(-gate[hd])) for hd in range(16)])
    y_ref = core.reshape(-1).astype(np.float32).astype(np.float16).astype(np.float64) @ wo.T
    assert np.allclose(y[0], y_ref, rtol=1e-9, atol=1e-9)
