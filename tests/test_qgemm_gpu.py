"""Prefill projection GEMMs (row f4: gemm_input / gemm of src/engine/weights.hip:306-330, the
kernels of kernels/qgemm.hpp) on MI355X through the C ABI.

- The activation prep equals the reference's CPU rule bit for bit (tests/test_qgemm.hip:188-196;
  oracle.qgemm_act_ref): f16 rounding and in-order 32-group sums.
- The GEMM is held to the reference's own bound (tests/test_qgemm.hip:140-166) against the
  float64 product of the same f16 activations with the oracle's dequantized rows:
  |y - W h| <= (K / 16 + 80) 2^-24 sum_k mag_k |h_k|, mag = 15 d sc + dmin m (Q4_K) or
  32 |d sc| (Q6_K).
Cases: the reference's fixture tensors (Q4_K K = 8192 N = 2, Q6_K K = 4096 N = 4, 70 tokens, as
tests/test_qgemm.hip:199-208), the attention's projections on random blocks (attn_q 2048 -> 8192,
attn_k 2048 -> 512, attn_output 4096 -> 2048, attn_v Q6_K 2048 -> 512) with token counts that
leave partial tiles, one token, a row stride ldy > n_rows with canaries past each row, and the
Python layer's reference error messages. Q4_K's 128-token tiles equal its 64 x 64 tiles bit for
bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from conftest import to_dev, to_host
from test_q4k_gpu import random_blocks, random_q6k_blocks

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
CANARY = -7777.0


def xs_normal(rng, n_tok, k, sigma=1.5):
    return (rng.standard_normal((n_tok, k)) * sigma).astype(np.float32)


def test_activation_prep_is_bit_identical_to_reference_rule(O, attn, torch_mod):
    torch = torch_mod
    rng = np.random.default_rng(3)
    for n_tok, k in ((70, 2048), (5, 4096), (1, 8192)):
        x = xs_normal(rng, n_tok, k)
        x[0, :32] = -1e-9  # a group of values that round to -0
        inp = attn.GemmInput(n_tok, k)
        attn.gemm_input(to_dev(torch, x.reshape(-1)), k, n_tok, inp)
        torch.cuda.synchronize()
        h, s = O.qgemm_act_ref(x)
        got_h = to_host(inp.xh)[:n_tok * k]
        got_s = to_host(inp.xs)[:n_tok * k // 32]
        assert np.array_equal(got_h, h.view(np.uint16))
        assert np.array_equal(got_s.view(np.uint32), s.view(np.uint32))


def test_activation_prep_matches_the_reference_kernel(O, attn, torch_mod, ref_kernels):
    """Pins qgemm_act_ref and this repository's gemm_input against the reference's own
    qgemm_act_kernel (kernels/qgemm.hpp:40-60), built from its sources into oracle/_ref and
    launched with the engine's shape (src/engine/weights.hip:310-312): xh and xs bit for bit, on
    the same shapes and values as the test above, the group that rounds to -0 included."""
    if ref_kernels is None:
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    torch = torch_mod
    rng = np.random.default_rng(3)
    for n_tok, k in ((70, 2048), (5, 4096), (1, 8192)):
        x = xs_normal(rng, n_tok, k)
        x[0, :32] = -1e-9  # a group of values that round to -0
        xd = to_dev(torch, x.reshape(-1))
        ref_h = torch.empty(n_tok * k, dtype=torch.float16, device="cuda")
        ref_s = torch.empty(n_tok * k // 32, dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        assert ref_kernels.ref_qgemm_act(xd.data_ptr(), ref_h.data_ptr(), ref_s.data_ptr(), k,
                                         n_tok) == 0
        inp = attn.GemmInput(n_tok, k)
        attn.gemm_input(xd, k, n_tok, inp)
        torch.cuda.synchronize()
        rh, rs = to_host(ref_h), to_host(ref_s)
        h, s = O.qgemm_act_ref(x)
        assert np.array_equal(rh, h.view(np.uint16)), "oracle rule vs the reference kernel (xh)"
        assert np.array_equal(rs.view(np.uint32), s.view(np.uint32)), "oracle rule (xs)"
        assert np.array_equal(to_host(inp.xh)[:n_tok * k], rh), "gemm_input vs reference (xh)"
        assert np.array_equal(to_host(inp.xs)[:n_tok * k // 32].view(np.uint32),
                              rs.view(np.uint32)), "gemm_input vs reference (xs)"
        # -0 halves, and a +0 sum: the sum starts at +0 and +0 + -0 = +0
        assert rh[:32].tolist() == [0x8000] * 32 and rs.view(np.uint32)[0] == 0


def run_gemm(O, attn, torch, fmt, blocks, n, k, x, ldy):
    n_tok = x.shape[0]
    inp = attn.GemmInput(n_tok, k)
    attn.gemm_input(to_dev(torch, x.reshape(-1)), k, n_tok, inp)
    r1 = O.q4k_repack_r1(blocks) if fmt == "q4_k" else O.q6k_repack_r1(blocks, n, k)
    y = torch.full((n_tok * ldy,), CANARY, dtype=torch.float32, device="cuda")
    attn.gemm(to_dev(torch, r1), fmt, n, k, inp, y, ldy)
    torch.cuda.synchronize()
    out = to_host(y).reshape(n_tok, ldy)
    assert (out[:, n:] == CANARY).all(), "write past n_rows"
    return out[:, :n].astype(np.float64)


def magnitudes(O, fmt, blocks, n, k):
    if fmt == "q4_k":
        w, ds = O.q4k_dequant(blocks)
        mag = 15.0 * ds.astype(np.float64) + O.q4k_mins(blocks)
    else:
        w = O.q6k_dequant(blocks)
        blk = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 210)
        d = blk[:, 208:210].copy().view(np.float16).astype(np.float64).reshape(-1)
        sc = blk[:, 192:208].view(np.int8).astype(np.float64)
        mag = np.repeat(np.abs(32.0 * d[:, None] * sc), 16, axis=1).reshape(-1)
    return w.reshape(n, k).astype(np.float64), mag.reshape(n, k)


def check(O, attn, torch, fmt, blocks, n, k, x, name, ldy_pad=3):
    got = run_gemm(O, attn, torch, fmt, blocks, n, k, x, n + ldy_pad)
    w, mag = magnitudes(O, fmt, blocks, n, k)
    h = x.astype(np.float16).astype(np.float64)
    ref = h @ w.T
    bound = (k / 16.0 + 80.0) * 2.0 ** -24 * (np.abs(h) @ mag.T) + 1e-30
    ratio = np.abs(got - ref) / bound
    print(f"[qgemm {name} {fmt}] N={n} K={k} tokens={x.shape[0]} max err/bound "
          f"{ratio.max():.3f}", flush=True)
    assert np.isfinite(got).all()
    assert (ratio <= 1.0).all(), np.unravel_index(int(ratio.argmax()), ratio.shape)


def test_reference_fixtures(O, attn, torch_mod):
    g4 = np.load(GOLDEN / "q4k_tiny.npz")
    k, n = int(g4["k"]), int(g4["n"])
    check(O, attn, torch_mod, "q4_k", g4["blocks"], n, k,
          xs_normal(np.random.default_rng(5), 70, k), "fixture")
    g6 = np.load(GOLDEN / "q6k_tiny.npz")
    k, n = int(g6["k"]), int(g6["n"])
    check(O, attn, torch_mod, "q6_k", g6["blocks"], n, k,
          xs_normal(np.random.default_rng(6), 70, k), "fixture")


@pytest.mark.parametrize("k,n,n_tok", [(2048, 8192, 130), (2048, 512, 70), (4096, 2048, 200),
                                       (2048, 1001, 129), (4096, 37, 1), (8192, 100, 65),
                                       (2048, 2048, 2048)])
def test_q4k_shapes(O, attn, torch_mod, k, n, n_tok):
    rng = np.random.default_rng(k + 7 * n + n_tok)
    check(O, attn, torch_mod, "q4_k", random_blocks(rng, n, k), n, k, xs_normal(rng, n_tok, k),
          "random")


@pytest.mark.parametrize("k,n,n_tok", [(2048, 512, 130), (2048, 37, 65), (4096, 300, 3)])
def test_q6k_shapes(O, attn, torch_mod, k, n, n_tok):
    rng = np.random.default_rng(3 * k + n + n_tok)
    check(O, attn, torch_mod, "q6_k", random_q6k_blocks(rng, n, k), n, k, xs_normal(rng, n_tok, k),
          "random")


@pytest.mark.parametrize("k,n,n_tok", [(2048, 8192, 600), (2048, 2000, 2100), (4096, 2048, 2048)])
def test_q4k_token_tiles_bit_identical(O, attn, torch_mod, k, n, n_tok):
    """Q4_K runs 128 x 128 tiles (qgemm_q4k_big_kernel) when they give every CU one, as in every
    case here (the last token tile partial in the first two, the last row tile in the second; the
    third is attn_output's shape, k = 4096); at most 64 tokens always run 64 x 64 tiles
    (qgemm_kernel). Each output element is the same arithmetic in the same order either way, so
    the product equals, bit for bit, the same product computed 64 tokens at a time."""
    torch = torch_mod
    rng = np.random.default_rng(k + n + n_tok)
    r1 = to_dev(torch, O.q4k_repack_r1(random_blocks(rng, n, k)))
    x = xs_normal(rng, n_tok, k)
    ldy = n + 3

    def product(xc):
        inp = attn.GemmInput(xc.shape[0], k)
        attn.gemm_input(to_dev(torch, xc.reshape(-1)), k, xc.shape[0], inp)
        y = torch.full((xc.shape[0] * ldy,), CANARY, dtype=torch.float32, device="cuda")
        attn.gemm(r1, "q4_k", n, k, inp, y, ldy)
        torch.cuda.synchronize()
        return to_host(y).reshape(xc.shape[0], ldy)

    whole = product(x)
    parts = np.concatenate([product(x[t:t + 64]) for t in range(0, n_tok, 64)])
    print(f"[qgemm tiles] N={n} K={k} tokens={n_tok}: "
          f"{int((whole != parts).sum())} elements differ", flush=True)
    assert (whole[:, n:] == CANARY).all(), "write past n_rows"
    assert np.isfinite(whole[:, :n]).all()
    assert np.array_equal(whole, parts)


def test_full_row_stride_and_tile_edges(O, attn, torch_mod):
    """n_rows and n_tok exact multiples of the 64 x 64 tile, ldy == n_rows (no padding)."""
    rng = np.random.default_rng(17)
    k, n, n_tok = 2048, 128, 128
    blocks = random_blocks(rng, n, k)
    check(O, attn, torch_mod, "q4_k", blocks, n, k, xs_normal(rng, n_tok, k), "exact", ldy_pad=0)


def test_python_layer_reference_errors(attn, torch_mod):
    torch = torch_mod
    inp = attn.GemmInput(4, 2048)
    x = torch.zeros(8 * 2048, device="cuda")
    with pytest.raises(RuntimeError, match="gemm_input: chunk does not fit"):
        attn.gemm_input(x, 2048, 8, inp)
    with pytest.raises(RuntimeError, match="gemm_input: chunk does not fit"):
        attn.gemm_input(x, 1000, 4, inp)
    attn.gemm_input(x, 2048, 4, inp)
    w = torch.zeros(8 * 2048 // 256 * 144, dtype=torch.uint8, device="cuda")
    y = torch.zeros(4 * 8, device="cuda")
    with pytest.raises(RuntimeError, match="gemm: K mismatch"):
        attn.gemm(w, "q4_k", 8, 4096, inp, y, 8)
    with pytest.raises(RuntimeError, match="gemm: unsupported type"):
        attn.gemm(w, "q8_0", 8, 2048, inp, y, 8)
