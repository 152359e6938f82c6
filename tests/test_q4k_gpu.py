"""Q4_K and Q6_K GEMVs (row f4) on MI355X through the C ABI, against the oracle's float64 product
over the reference-dequantized rows, with the per-row error bound of the reference's own test
(tests/test_q4k_gemv.hip:60-113; oracle.q4k_error_bound): |y - W x| <= sum |W| e(x) +
K 2^-23 sum |W x| (+ the fp16 nibble-chain term). Cases: the reference's fixture (real model
blocks, K = 8192, N = 2), the engine's attention projections (attn_q 2048 -> 8192, attn_k
2048 -> 512, attn_output 4096 -> 2048) on random blocks, row counts that leave a partial last
step, an activation whose products cancel, and a canary past n_rows.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import to_dev, to_host

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "q4k_tiny.npz"
CANARY = -7777.0


def random_blocks(rng, n_rows, k):
    nb = n_rows * k // 256
    b = rng.integers(0, 256, (nb, 144), dtype=np.uint8)
    d = (rng.random(nb) * 0.01 + 1e-4).astype(np.float16)
    dmin = (rng.random(nb) * 0.005 + 1e-5).astype(np.float16)
    b[:, 0:2] = d.view(np.uint8).reshape(nb, 2)
    b[:, 2:4] = dmin.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def run(O, attn, torch, blocks, x, n_rows, k, act):
    r1 = O.q4k_repack_r1(blocks)
    y = torch.full((n_rows + 64,), CANARY, dtype=torch.float32, device="cuda")
    attn.q4k_gemv(to_dev(torch, r1), to_dev(torch, x.astype(np.float32)), y, n_rows, k, act)
    torch.cuda.synchronize()
    out = to_host(y)
    assert (out[n_rows:] == CANARY).all(), "write past n_rows"
    return out[:n_rows].astype(np.float64)


def check(O, attn, torch, blocks, x, n_rows, k, act, name):
    got = run(O, attn, torch, blocks, x, n_rows, k, act)
    ref = O.q4k_gemv_f64(blocks, x, n_rows, k)
    w, ds = O.q4k_dequant(blocks)
    bound = O.q4k_error_bound(w.reshape(n_rows, k), ds.reshape(n_rows, k), x, act)
    ratio = np.abs(got - ref) / bound
    print(f"[q4k {name} {act}] N={n_rows} K={k} max err/bound {ratio.max():.3f} "
          f"max abs {np.abs(got - ref).max():.3e}", flush=True)
    assert np.isfinite(got).all()
    assert (ratio <= 1.0).all(), (int(ratio.argmax()), got[ratio.argmax()], ref[ratio.argmax()])


@pytest.mark.parametrize("act", ["fp16", "int8"])
def test_reference_fixture(O, attn, torch_mod, act):
    g = np.load(GOLDEN)
    k, n = int(g["k"]), int(g["n"])
    x = np.random.default_rng(7).standard_normal(k).astype(np.float32) * 1.5
    check(O, attn, torch_mod, g["blocks"], x, n, k, act, "fixture")


@pytest.mark.parametrize("k,n", [(2048, 8192), (2048, 512), (4096, 2048), (2048, 1001),
                                 (4096, 37), (8192, 300)])
@pytest.mark.parametrize("act", ["fp16", "int8"])
def test_engine_shapes(O, attn, torch_mod, k, n, act):
    rng = np.random.default_rng(k + n)
    blocks = random_blocks(rng, n, k)
    x = rng.standard_normal(k).astype(np.float32)
    check(O, attn, torch_mod, blocks, x, n, k, act, "random")


def test_cancelling_activation(O, attn, torch_mod):
    """An o-proj input with a wide dynamic range and sign structure, so row outputs cancel."""
    rng = np.random.default_rng(11)
    k, n = 4096, 2048
    blocks = random_blocks(rng, n, k)
    x = (rng.standard_normal(k) * np.exp(rng.standard_normal(k) * 2)).astype(np.float32)
    x[::2] = -np.abs(x[::2])
    x[1::2] = np.abs(x[1::2])
    for act in ("fp16", "int8"):
        check(O, attn, torch_mod, blocks, x, n, k, act, "cancel")


# ------------------------------------------------------------------------------------------------
# Q6_K (attn_v): the same bound with d sc replaced by d |sc| and codes q - 32 (|q - 32| <= 32):
# activation error times |W|, K 2^-23 sum |W x| of accumulation, and the f16 chain term
# 2^-20 * 63 * d |sc| |x| (codes up to 63 accumulate in 16-element chains before scaling).
# ------------------------------------------------------------------------------------------------

Q6K_GOLDEN = Path(__file__).resolve().parent / "golden" / "q6k_tiny.npz"


def random_q6k_blocks(rng, n_rows, k):
    nb = n_rows * k // 256
    b = rng.integers(0, 256, (nb, 210), dtype=np.uint8)
    d = (rng.random(nb) * 0.004 + 1e-4).astype(np.float16)
    b[:, 208:210] = d.view(np.uint8).reshape(nb, 2)
    return b.reshape(-1)


def q6k_check(O, attn, torch, blocks, x, n, k, name):
    r1 = O.q6k_repack_r1(blocks, n, k)
    y = torch.full((n + 64,), CANARY, dtype=torch.float32, device="cuda")
    attn.q6k_gemv(to_dev(torch, r1), to_dev(torch, x.astype(np.float32)), y, n, k)
    torch.cuda.synchronize()
    out = to_host(y)
    assert (out[n:] == CANARY).all(), "write past n_rows"
    got = out[:n].astype(np.float64)
    ref = O.q6k_gemv_f64(blocks, x, n, k)
    w = O.q6k_dequant(blocks).reshape(n, k).astype(np.float64)
    nb = k // 256
    blk = blocks.reshape(n * nb, 210)
    d = blk[:, 208:210].copy().view(np.float16).astype(np.float64).reshape(-1)
    sc = blk[:, 192:208].view(np.int8).astype(np.float64)
    dsc = np.repeat(np.abs(d[:, None] * sc), 16, axis=1).reshape(n, k)
    x64 = x.astype(np.float64)
    e = np.abs(x64) * 2.0 ** -11 + 2.0 ** -25
    bound = (np.abs(w) @ e + k * 2.0 ** -23 * (np.abs(w) @ np.abs(x64))
             + 2.0 ** -20 * 63.0 * (dsc @ np.abs(x64)))
    ratio = np.abs(got - ref) / bound
    print(f"[q6k {name}] N={n} K={k} max err/bound {ratio.max():.3f}", flush=True)
    assert np.isfinite(got).all() and (ratio <= 1.0).all(), int(ratio.argmax())


def test_q6k_reference_fixture(O, attn, torch_mod):
    g = np.load(Q6K_GOLDEN)
    k, n = int(g["k"]), int(g["n"])
    x = np.random.default_rng(9).standard_normal(k).astype(np.float32) * 1.5
    q6k_check(O, attn, torch_mod, g["blocks"], x, n, k, "fixture")


@pytest.mark.parametrize("k,n", [(2048, 512), (2048, 8192), (4096, 1001), (8192, 37)])
def test_q6k_shapes(O, attn, torch_mod, k, n):
    rng = np.random.default_rng(3 * k + n)
    q6k_check(O, attn, torch_mod, random_q6k_blocks(rng, n, k),
              rng.standard_normal(k).astype(np.float32), n, k, "random")


@pytest.mark.parametrize("n4,n6", [(8192, 512), (1001, 37), (16, 3000)])
def test_pair_matches_separate_launches(O, attn, torch_mod, n4, n6):
    """One mixed launch (attn_q Q4_K + attn_v Q6_K, K = 2048) equals the two separate launches
    bit for bit, and both outputs stay inside their oracle bounds (checked by the separate
    tests on the same kernels)."""
    torch = torch_mod
    k = 2048
    rng = np.random.default_rng(n4 + 7 * n6)
    b4, b6 = random_blocks(rng, n4, k), random_q6k_blocks(rng, n6, k)
    x = to_dev(torch, rng.standard_normal(k).astype(np.float32))
    w4, w6 = to_dev(torch, O.q4k_repack_r1(b4)), to_dev(torch, O.q6k_repack_r1(b6, n6, k))
    y4 = torch.full((n4 + 64,), CANARY, device="cuda")
    y6 = torch.full((n6 + 64,), CANARY, device="cuda")
    s4, s6 = torch.empty(n4, device="cuda"), torch.empty(n6, device="cuda")
    attn.q4k_q6k_gemv_pair(w4, n4, y4, w6, n6, y6, x)
    attn.q4k_gemv(w4, x, s4, n4, k, "fp16")
    attn.q6k_gemv(w6, x, s6, n6, k)
    torch.cuda.synchronize()
    assert torch.equal(y4[:n4], s4) and torch.equal(y6[:n6], s6)
    assert (to_host(y4)[n4:] == CANARY).all() and (to_host(y6)[n6:] == CANARY).all()
    ref = O.q4k_gemv_f64(b4, to_host(x), n4, k)
    assert np.abs(to_host(s4) - ref).max() <= 1e-3 * np.abs(ref).max() + 1e-3


@pytest.mark.parametrize("nq,nk,nv", [(8192, 512, 512), (100, 3000, 7)])
def test_qkv_one_launch_matches_separate(O, attn, torch_mod, nq, nk, nv):
    """q, k (Q4_K) and v (Q6_K) in one launch equal the three separate launches bit for bit."""
    torch = torch_mod
    k = 2048
    rng = np.random.default_rng(nq + 3 * nk + 5 * nv)
    bq, bk, bv = random_blocks(rng, nq, k), random_blocks(rng, nk, k), random_q6k_blocks(rng, nv, k)
    x = to_dev(torch, rng.standard_normal(k).astype(np.float32))
    wq, wk = to_dev(torch, O.q4k_repack_r1(bq)), to_dev(torch, O.q4k_repack_r1(bk))
    wv = to_dev(torch, O.q6k_repack_r1(bv, nv, k))
    ys = [torch.full((n + 64,), CANARY, device="cuda") for n in (nq, nk, nv)]
    ss = [torch.empty(n, device="cuda") for n in (nq, nk, nv)]
    attn.qkv_gemv(wq, nq, ys[0], wk, nk, ys[1], wv, nv, ys[2], x)
    attn.q4k_gemv(wq, x, ss[0], nq, k, "fp16")
    attn.q4k_gemv(wk, x, ss[1], nk, k, "fp16")
    attn.q6k_gemv(wv, x, ss[2], nv, k)
    torch.cuda.synchronize()
    for y, s_, n in zip(ys, ss, (nq, nk, nv)):
        assert torch.equal(y[:n], s_)
        assert (to_host(y)[n:] == CANARY).all()
