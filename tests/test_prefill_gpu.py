"""Causal prefill parity on MI355X: the MFMA flash kernel (through the C ABI) against the FP64
oracle.

Mirrors the reference's check_prefill list (tests/test_attn_splitk.hip:271-279: partial 4-token
blocks, a 32-key sub-chunk crossing, a non-empty prefix) with q = 2 N(0,1), then the BASELINE
configs C3 (2048 tokens, empty cache; every row) and C4 (8192 tokens after an 8192-token prefix;
a deterministic row sample covering first/last tiles and diagonal tiles), plus two size-free
properties: chunked prefill equals one-shot prefill, and prefill row t equals decode at pos0+t+1.
The balanced form (miso_attn_prefill_ws: heavy token blocks split between two workgroups, the
parts merged through a workspace; 16-token blocks up to 2048 tokens, 32-token blocks from 3841
to 4096)
is checked the same way, on shapes with and without split blocks, plus run-to-run bit equality
and reuse of one workspace across sizes.
Gate: |got - ref| <= 2e-3 + 1e-2 |ref| for every element (f32 output).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, D = 16, 256


def run_prefill(attn, torch, p, pos0=None, n=None, t_from=0, scratch=None):
    """Prefill tokens [t_from, t_from + n) of the case (positions pos0 + t); with `scratch`, the
    balanced form."""
    pos0 = p["pos0"] if pos0 is None else pos0
    n = p["n"] if n is None else n
    S = p["qg_stride"]
    q = to_dev(torch, p["q"][t_from * H * D:(t_from + n) * H * D])
    qg = to_dev(torch, p["qg"][t_from * S:(t_from + n) * S])
    k, v = to_dev(torch, p["k"]), to_dev(torch, p["v"])
    core = torch.full((n * H * D,), -1.0, device="cuda")
    attn.attn_prefill(q, qg, k, v, core, pos0, n, p["max_ctx"], S, scratch=scratch)
    torch.cuda.synchronize()
    return to_host(core).reshape(n, H, D)


def check(O, attn, torch, pos0, n, q_scale=2.0, seed=None, rows=None, name="prefill",
          max_ctx=None, scratch=None):
    p = O.prefill_inputs(1000 + 17 * pos0 + n if seed is None else seed, pos0, n,
                         max_ctx if max_ctx else pos0 + n + 5, q_scale=q_scale)
    got = run_prefill(attn, torch, p, scratch=scratch)
    rows = np.arange(n) if rows is None else np.asarray(rows)
    ref = O.prefill_f64(p["q"], p["qg"], p["qg_stride"], p["k"], p["v"], pos0, p["max_ctx"], rows)
    st = O.compare(got[rows], ref)
    report(f"{name} pos0={pos0} n={n} rows={rows.size}", st)
    assert st["ok"], st
    return p, got


@pytest.mark.parametrize("pos0,n", [(0, 1), (0, 3), (0, 4), (0, 5), (0, 33), (40, 17), (0, 128),
                                    (5, 100), (100, 16), (31, 47)])
def test_prefill_matches_oracle(O, attn, torch_mod, pos0, n):
    check(O, attn, torch_mod, pos0, n)


def test_prefill_c3_all_rows(O, attn, torch_mod):
    """C3: 2048 tokens, empty cache, q/K/V ~ N(0,1) from seed 2048."""
    check(O, attn, torch_mod, 0, 2048, q_scale=1.0, seed=2048, max_ctx=2048, name="C3")


def c4_rows(n=8192, block=16):
    rng = np.random.default_rng(16384)
    fixed = [0, 1, 15, 16, 31, 32, 33, 1023, 1024, 4095, 4096, 8176, 8190, 8191]
    diag = [b * block + r for b in (7, 300, 511) for r in (0, 3, 4, 7, 8, 15)]
    rand = rng.choice(n, 96, replace=False).tolist()
    return np.unique(np.array(fixed + diag + rand))


def test_prefill_c4_sampled_rows(O, attn, torch_mod):
    """C4: 8192 new tokens after an 8192-token prefix (total 16384 keys), seed 16384."""
    check(O, attn, torch_mod, 8192, 8192, q_scale=1.0, seed=16384, max_ctx=16384,
          rows=c4_rows(), name="C4")


def test_prefill_chunked_equals_one_shot(O, attn, torch_mod):
    torch = torch_mod
    p = O.prefill_inputs(4242, 0, 300, 300, q_scale=1.0)
    whole = run_prefill(attn, torch, p)
    a = run_prefill(attn, torch, p, pos0=0, n=100, t_from=0)
    b = run_prefill(attn, torch, p, pos0=100, n=200, t_from=100)
    st = O.compare(np.concatenate([a, b]), whole.astype(np.float64))
    assert st["ok"], st


def test_prefill_rows_equal_decode(O, attn, torch_mod):
    torch = torch_mod
    pos0, n = 1000, 40
    p = O.prefill_inputs(99, pos0, n, pos0 + n, q_scale=1.0)
    rows = run_prefill(attn, torch, p)
    k, v = to_dev(torch, p["k"]), to_dev(torch, p["v"])
    sc = attn.DecodeScratch(128)
    for t in (0, 17, 39):
        q = to_dev(torch, p["q"][t * H * D:(t + 1) * H * D])
        qg = to_dev(torch, p["qg"][t * p["qg_stride"]: t * p["qg_stride"] + H * 2 * D])
        core = torch.empty(H * D, device="cuda")
        attn.attn_decode(q, qg, k, v, core, sc, pos0 + t + 1, p["max_ctx"])
        torch.cuda.synchronize()
        st = O.compare(rows[t], to_host(core).reshape(H, D).astype(np.float64))
        assert st["ok"], (t, st)


def test_prefill_engine_stride(O, attn, torch_mod):
    """qg_stride 9216: the engine's shared [q+gate | k | v] projection rows."""
    p = O.prefill_inputs(9216, 64, 50, 120, q_scale=2.0, qg_stride=9216)
    got = run_prefill(attn, torch_mod, p)
    ref = O.prefill_f64(p["q"], p["qg"], 9216, p["k"], p["v"], 64, 120, np.arange(50))
    st = O.compare(got, ref)
    assert st["ok"], st


def test_reference_prefill_kernel_agrees_with_oracle(O, attn, torch_mod, ref_kernels):
    """Second checker: the reference's own prefill kernel (built from its sources) reproduces
    the oracle within the reference's rel-L2 gate of 1e-5 (test_attn_splitk.hip:267)."""
    if ref_kernels is None:
        pytest.skip("oracle/_ref not built (needs the reference tree at build time)")
    torch = torch_mod
    for pos0, n in ((0, 5), (40, 17)):
        p = O.prefill_inputs(1000 + 17 * pos0 + n, pos0, n, pos0 + n + 5, q_scale=2.0)
        q, qg = to_dev(torch, p["q"]), to_dev(torch, p["qg"])
        k, v = to_dev(torch, p["k"]), to_dev(torch, p["v"])
        core = torch.full((n * H * D,), -1.0, device="cuda")
        torch.cuda.synchronize()
        assert ref_kernels.ref_attn_prefill(q.data_ptr(), qg.data_ptr(), k.data_ptr(),
                                            v.data_ptr(), core.data_ptr(), pos0, n,
                                            p["max_ctx"], p["qg_stride"]) == 0
        torch.cuda.synchronize()
        got = to_host(core).reshape(n, H, D)
        ref = O.prefill_f64(p["q"], p["qg"], p["qg_stride"], p["k"], p["v"], pos0, p["max_ctx"],
                            np.arange(n))
        rel = np.sqrt(((got - ref) ** 2).sum(axis=2) / (ref ** 2).sum(axis=2)).max()
        assert rel <= 1e-5, rel


@pytest.fixture(scope="module")
def prefill_scratch(attn, torch_mod):
    return attn.PrefillScratch()


def balanced_rows(pos0, n):
    """Every row up to 1200 tokens; else the first and last rows of every 64th block, the last
    128 rows (the heaviest blocks, split) and a seeded sample."""
    if n <= 1200:
        return None
    rng = np.random.default_rng(n + pos0)
    rows = [b * 16 + r for b in range(0, (n + 15) // 16, 64) for r in (0, 15)]
    rows += list(range(max(0, n - 128), n)) + rng.choice(n, 64, replace=False).tolist()
    return np.unique(np.array([r for r in rows if r < n]))


@pytest.mark.parametrize("pos0,n", [(0, 1), (0, 16), (0, 17), (0, 48), (0, 129), (0, 300),
                                    (7, 999), (100, 1500), (3000, 600), (1, 2047), (0, 2049),
                                    (0, 3841), (500, 4000), (0, 4096), (4096, 4096)])
def test_prefill_balanced_matches_oracle(O, attn, torch_mod, prefill_scratch, pos0, n):
    check(O, attn, torch_mod, pos0, n, rows=balanced_rows(pos0, n), name="balanced",
          scratch=prefill_scratch)


def test_prefill_balanced_c3_all_rows(O, attn, torch_mod, prefill_scratch):
    """C3 through the balanced form: 2048 tokens, empty cache, every row."""
    check(O, attn, torch_mod, 0, 2048, q_scale=1.0, seed=2048, max_ctx=2048, name="C3 balanced",
          scratch=prefill_scratch)


def test_prefill_balanced_repeatable(O, attn, torch_mod, prefill_scratch):
    """Bit-equal across calls (the merge does not depend on which part arrives second), one
    workspace across sizes and across the 16- and 32-token block layouts (whose partial regions
    differ), and within the gate of the one-block-per-workgroup form."""
    torch = torch_mod
    p = O.prefill_inputs(777, 0, 2048, 2048, q_scale=1.0)
    first = run_prefill(attn, torch, p, scratch=prefill_scratch)
    small = O.prefill_inputs(778, 40, 333, 400, q_scale=2.0)
    a = run_prefill(attn, torch, small, scratch=prefill_scratch)
    wide = O.prefill_inputs(779, 0, 4096, 4096, q_scale=1.0)
    w = run_prefill(attn, torch, wide, scratch=prefill_scratch)
    for _ in range(3):
        again = run_prefill(attn, torch, p, scratch=prefill_scratch)
        assert np.array_equal(again, first)
        assert np.array_equal(run_prefill(attn, torch, wide, scratch=prefill_scratch), w)
    assert np.array_equal(run_prefill(attn, torch, small, scratch=prefill_scratch), a)
    plain = run_prefill(attn, torch, p)
    st = O.compare(first, plain.astype(np.float64))
    report("balanced vs plain C3 inputs", st)
    assert st["ok"], st
    assert not np.array_equal(first, plain)  # the split blocks did merge two parts


@pytest.mark.parametrize("n", [2049, 3840, 4097])
def test_prefill_balanced_wide_is_plain(O, attn, torch_mod, prefill_scratch, n):
    """Outside the balanced form's sizes the balanced entry runs the one-workgroup-per-block
    layout, bit-equal to miso_attn_prefill."""
    torch = torch_mod
    p = O.prefill_inputs(n, 0, n, n, q_scale=1.0)
    assert attn.prefill_workspace_bytes(n) == 0
    assert np.array_equal(run_prefill(attn, torch, p, scratch=prefill_scratch),
                          run_prefill(attn, torch, p))
