"""CPU pins of the oracle's Q4_K and Q6_K functions (oracle/attn_oracle.c: oracle_q4k_*,
oracle_q6k_*), which restate the reference's GGUF dequantization (src/dequant.cpp:45-75,80-84),
its r1 repacks (src/repack.cpp:9-25,53-74) and its GEMV reference (tests/test_q4k_gemv.hip:80-90);
Q6_K below the Q4_K tests, with the same kinds of pins:

  * dequant: bit-identical to the reference's own dequantized fixture (tests/fixtures/
    tiny.q4_k.f32, K = 8192, N = 2, real model blocks; tests/golden/q4k_tiny.npz);
  * dequant on synthetic blocks: each weight equals d sc q - dmin m recomputed from fields set
    by hand (6-bit scale / min packing of all 8 sub-blocks, nibble order);
  * repack: bytes outside 4..15 unchanged, and the 24-bit fields decode to the GGUF scale / min
    pairs;
  * GEMV: equal to numpy's float64 product over the dequantized rows.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "q4k_tiny.npz"


def test_dequant_matches_reference_fixture():
    g = np.load(GOLDEN)
    w, _ = O.q4k_dequant(g["blocks"])
    assert np.array_equal(w.view(np.uint32), g["dequant"].astype(np.float32).view(np.uint32))


def pack_block(d, dmin, sc, m, q):
    """A GGUF Q4_K block from fields: sc, m [8] 6-bit, q [256] 4-bit."""
    b = np.zeros(144, np.uint8)
    b[0:2] = np.frombuffer(np.float16(d).tobytes(), np.uint8)
    b[2:4] = np.frombuffer(np.float16(dmin).tobytes(), np.uint8)
    s = np.zeros(12, np.uint8)
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= m[j] & 63
        else:
            s[j + 4] |= (sc[j] & 15) | ((m[j] & 15) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (m[j] >> 4) << 6
    b[4:16] = s
    for j in range(8):
        for l in range(32):
            b[16 + 32 * (j // 2) + l] |= (q[32 * j + l] & 15) << (4 * (j % 2))
    return b


def test_dequant_fields_closed_form():
    rng = np.random.default_rng(3)
    blocks, want = [], []
    for _ in range(6):
        d, dmin = np.float16(rng.random() * 0.02), np.float16(rng.random() * 0.01)
        sc, m = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
        q = rng.integers(0, 16, 256)
        blocks.append(pack_block(d, dmin, sc, m, q))
        for j in range(8):
            dj = np.float32(np.float32(d) * np.float32(sc[j]))
            mj = np.float32(np.float32(dmin) * np.float32(m[j]))
            want.extend(np.float32(dj * np.float32(q[32 * j + l]) - mj) for l in range(32))
    w, ds = O.q4k_dequant(np.concatenate(blocks))
    assert np.array_equal(w, np.array(want, np.float32))


def test_repack_r1_fields():
    g = np.load(GOLDEN)
    src = g["blocks"].reshape(-1, 144)
    r1 = O.q4k_repack_r1(src).reshape(-1, 144)
    assert np.array_equal(r1[:, :4], src[:, :4]) and np.array_equal(r1[:, 16:], src[:, 16:])
    w, ds = O.q4k_dequant(src)
    for b in range(src.shape[0]):
        for gi in range(4):
            v = int(r1[b, 4 + 3 * gi]) | int(r1[b, 5 + 3 * gi]) << 8 | int(r1[b, 6 + 3 * gi]) << 16
            sc0, m0, sc1, m1 = v & 63, (v >> 6) & 63, (v >> 12) & 63, (v >> 18) & 63
            d = np.float32(np.frombuffer(src[b, 0:2].tobytes(), np.float16)[0])
            assert ds[b * 256 + 64 * gi] == np.float32(d * np.float32(sc0))
            assert ds[b * 256 + 64 * gi + 32] == np.float32(d * np.float32(sc1))
            dmin = np.float32(np.frombuffer(src[b, 2:4].tobytes(), np.float16)[0])
            # a weight with nibble 0 is exactly -dmin m
            for j, mm in ((2 * gi, m0), (2 * gi + 1, m1)):
                nib = (src[b, 16 + 32 * gi:16 + 32 * gi + 32] >> (4 * (j % 2))) & 15
                zero = np.flatnonzero(nib == 0)
                if zero.size:
                    assert w[b * 256 + 32 * j + zero[0]] == -np.float32(dmin * np.float32(mm))


def test_gemv_equals_float64_product():
    g = np.load(GOLDEN)
    k, n = int(g["k"]), int(g["n"])
    x = np.random.default_rng(7).standard_normal(k).astype(np.float32) * 1.5
    w, _ = O.q4k_dequant(g["blocks"])
    y = O.q4k_gemv_f64(g["blocks"], x, n, k)
    np.testing.assert_allclose(y, w.reshape(n, k).astype(np.float64) @ x.astype(np.float64),
                               rtol=1e-12)


Q6K_GOLDEN = Path(__file__).resolve().parent / "golden" / "q6k_tiny.npz"


def test_q6k_dequant_matches_reference_fixture():
    """oracle_q6k_dequant (src/dequant.cpp:63-75) against the reference's dequantized fixture
    tests/fixtures/tiny.q6_k.f32 (K = 4096, N = 4)."""
    g = np.load(Q6K_GOLDEN)
    w = O.q6k_dequant(g["blocks"])
    assert np.array_equal(w.view(np.uint32), g["dequant"].astype(np.float32).view(np.uint32))


def test_q6k_repack_r1_sections():
    """r1 rows: per row the ql, qh, scale and d sections of its blocks in order, then zeros."""
    g = np.load(Q6K_GOLDEN)
    k, n = int(g["k"]), int(g["n"])
    nb = k // 256
    src = g["blocks"].reshape(n, nb, 210)
    r1 = O.q6k_repack_r1(g["blocks"], n, k).reshape(n, -1)
    assert r1.shape[1] == (nb * 210 + 15) // 16 * 16
    for r in range(n):
        assert np.array_equal(r1[r, :nb * 128], src[r, :, :128].reshape(-1))
        assert np.array_equal(r1[r, nb * 128:nb * 192], src[r, :, 128:192].reshape(-1))
        assert np.array_equal(r1[r, nb * 192:nb * 208], src[r, :, 192:208].reshape(-1))
        assert np.array_equal(r1[r, nb * 208:nb * 210], src[r, :, 208:210].reshape(-1))
        assert not r1[r, nb * 210:].any()


def test_q6k_gemv_equals_float64_product():
    g = np.load(Q6K_GOLDEN)
    k, n = int(g["k"]), int(g["n"])
    x = np.random.default_rng(8).standard_normal(k).astype(np.float32)
    w = O.q6k_dequant(g["blocks"])
    y = O.q6k_gemv_f64(g["blocks"], x, n, k)
    np.testing.assert_allclose(y, w.reshape(n, k).astype(np.float64) @ x.astype(np.float64),
                               rtol=1e-12)
