"""Q4_K GEMV (row f4) on MI355X through the C ABI, against the oracle's float64 product over the
reference-dequantized rows, with the per-row error bound of the reference's own test
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
