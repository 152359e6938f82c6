"""CPU pins of the oracle's e4m3 KV-row format (oracle/attn_oracle.c: oracle_e4m3_value,
oracle_e4m3_encode, oracle_fp8_encode_rows, oracle_decode_fp8_f64). The format has no reference
counterpart (the reference's cache is f16, src/engine/attention.hpp:35-41), so each function is
pinned against what the mathematics and an independent implementation fix:

  * code values: the OCP e4m3 closed form at named codes, monotonicity, f16 exactness;
  * the encoder (a nearest-code search): torch's own float32 -> float8_e4m3fn cast (round to
    nearest even) on random values and on every tie point;
  * row encoding: the scale is 2^(floor(log2 max|x|) - 7) by numpy's frexp, |x| / scale lands in
    [128, 256) for the row max, and every element is within half a code step;
  * decode over e4m3 rows: equal to the pinned f16 oracle (oracle_decode_f64) run on the
    dequantized rows, which are f16-exact for these scales.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as O


def test_code_values_closed_form():
    t = O.e4m3_table()
    assert t[0x38] == 1.0 and t[0x40] == 2.0 and t[0x30] == 0.5
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0  # largest finite
    assert t[0x01] == 2.0 ** -9 and t[0x07] == 7 * 2.0 ** -9  # subnormals
    assert t[0x08] == 2.0 ** -6  # smallest normal
    assert t[0x00] == 0.0 and np.signbit(t[0x80])
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    pos = t[:0x7F]
    assert np.all(np.diff(pos) > 0)  # codes 0..0x7E are increasing
    assert np.array_equal(t[0x80:0xFF], -pos)
    # every finite value is an f16 value (the kernel widens codes to f16 exactly)
    assert np.array_equal(pos.astype(np.float16).astype(np.float64), pos)


def test_encode_matches_torch_rne_cast():
    rng = np.random.default_rng(5)
    y = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 40,
        (rng.random(2000).astype(np.float32) - 0.5) * 0.05,  # subnormal range
        np.array([255.99, -255.99, 0.0, -1e-12], dtype=np.float32),
    ]).astype(np.float32)
    # tie points: midpoints between adjacent codes below 256
    vals = O.e4m3_table()[:0x79]
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    y = np.concatenate([y, mids, -mids])
    got = np.array([O.e4m3_encode(v) for v in y], dtype=np.uint8)
    want = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    # torch keeps the sign of values that round to zero, as the oracle does
    assert np.array_equal(got, want), np.flatnonzero(got != want)[:10]


def test_encode_rows_scale_and_error_bound():
    rng = np.random.default_rng(9)
    rows = np.concatenate([
        rng.standard_normal((64, 256)).astype(np.float32),
        rng.standard_normal((8, 256)).astype(np.float32) * 1e-3,
        rng.standard_normal((8, 256)).astype(np.float32) * 3e4,
        np.zeros((1, 256), np.float32),
    ])
    rows[3, 17] = 4.0  # the row max exactly a power of two
    codes, scales = O.fp8_encode_rows(rows)
    for r in range(rows.shape[0]):
        amax = np.abs(rows[r]).max()
        if amax == 0:
            assert scales[r] == 2.0 ** -107 and not codes[r].any()
            continue
        _, ex = np.frexp(amax)
        assert scales[r] == 2.0 ** (int(ex) - 1 - 7)
        assert 128 <= amax / scales[r] < 256
    deq = O.fp8_dequant(codes, scales)
    y = rows / scales[:, None].astype(np.float64)
    step = np.where(np.abs(y) < 2.0 ** -6, 2.0 ** -9, 2.0 ** (np.floor(np.log2(np.maximum(
        np.abs(y), 2.0 ** -6))) - 3))
    assert np.all(np.abs(deq / scales[:, None] - y) <= step / 2 + 1e-12)


@pytest.mark.parametrize("length", [1, 37, 512])
def test_decode_fp8_equals_f16_oracle_on_dequantized_rows(length):
    max_ctx = length + 3
    inp = O.decode_inputs(length, length, max_ctx)
    q, qg, k, v = inp["q"], inp["qg"], inp["k"], inp["v"]
    kf = O.f16_to_f32(k).reshape(2 * max_ctx, 256)
    vf = O.f16_to_f32(v).reshape(2 * max_ctx, 256)
    k8, ks = O.fp8_encode_rows(kf)
    v8, vs = O.fp8_encode_rows(vf)
    kd = O.fp8_dequant(k8, ks)
    vd = O.fp8_dequant(v8, vs)
    # N(0, 1) rows: scales 2^-6 .. 2^-5, so the dequantized rows are exact in f16
    k16 = O.f32_to_f16(kd.astype(np.float32))
    v16 = O.f32_to_f16(vd.astype(np.float32))
    assert np.array_equal(O.f16_to_f32(k16).astype(np.float64), kd)
    ref = O.decode_f64(q, qg, k16, v16, length, max_ctx)
    got = O.decode_fp8_f64(q, qg, k8, v8, ks, vs, length, max_ctx)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-13)
