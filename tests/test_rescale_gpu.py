"""The lazy-rescale paths against the FP64 oracle: key rows planted so that some heads' scores
jump by far more than the rescale slack (2^8) late in the sequence, several times, so that the
running max moves mid-stream -- in the middle of a decode split and of a prefill item, in
diagonal and in full tiles. With N(0, 1) inputs a move past the first tile is rare, so these
paths (the decode wave ballot and O rescale, the prefill's in-AGPR O rescale) need planted data.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REF_REL_L2, report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, KV, D, G = 16, 2, 256, 8


def plant(k, q_rows, kvh, max_ctx, pos, score, rng):
    """Row pos of KV head kvh := c * q_rows[h] for a random head h of the group, with c chosen
    so that head's score (q . k / 16, natural units) is about `score`; other heads see a random
    projection of it."""
    h = int(rng.integers(0, G))
    qv = q_rows[kvh * G + h].astype(np.float64)
    c = score * 16.0 / float(qv @ qv)
    row = (c * qv).astype(np.float16).view(np.uint16)
    at = (kvh * max_ctx + pos) * D
    k[at:at + D] = row


@pytest.mark.parametrize("length,n_splits", [(3000, 8), (777, 3), (40, 1)])
def test_decode_late_max_moves(O, attn, torch_mod, length, n_splits):
    d = O.decode_inputs(900 + length, length, length + 3, q_scale=1.0)
    rng = np.random.default_rng(length)
    q_rows = d["q"].reshape(H, D)
    k = d["k"].copy()
    for kvh in range(KV):
        # increasing spikes: each moves the running max by more than 2^8 (in log2 units)
        for j, frac in enumerate((0.2, 0.5, 0.8, 0.99)):
            plant(k, q_rows, kvh, d["max_ctx"], int(frac * (length - 1)), 8.0 + 9.0 * j, rng)
    d["k"] = k
    torch = torch_mod
    core = torch.full((H * D,), -9123.5, device="cuda")
    sc = attn.DecodeScratch(max(n_splits, 1))
    attn.attn_decode(to_dev(torch, d["q"]), to_dev(torch, d["qg"]), to_dev(torch, d["k"]),
                     to_dev(torch, d["v"]), core, sc, length, d["max_ctx"], n_splits)
    torch.cuda.synchronize()
    got = to_host(core).reshape(H, D)
    ref = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], length, d["max_ctx"])
    st = O.compare(got, ref)
    report(f"decode rescale len={length} splits={n_splits}", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st


@pytest.mark.parametrize("pos0,n", [(0, 300), (1000, 64), (37, 50)])
def test_prefill_late_max_moves(O, attn, torch_mod, pos0, n):
    p = O.prefill_inputs(700 + pos0 + n, pos0, n, pos0 + n + 2, q_scale=1.0)
    rng = np.random.default_rng(pos0 + 3 * n)
    q = p["q"].reshape(n, H, D)
    k = p["k"].copy()
    kv_end = pos0 + n
    for kvh in range(KV):
        for j, frac in enumerate((0.1, 0.35, 0.6, 0.9)):
            pos = int(frac * (kv_end - 1))
            t = int(rng.integers(max(0, pos - pos0), n)) if pos >= pos0 else int(rng.integers(0, n))
            plant(k, q[t], kvh, p["max_ctx"], pos, 8.0 + 9.0 * j, rng)
    p["k"] = k
    torch = torch_mod
    S = p["qg_stride"]
    core = torch.full((n * H * D,), -1.0, device="cuda")
    attn.attn_prefill(to_dev(torch, p["q"]), to_dev(torch, p["qg"]), to_dev(torch, p["k"]),
                      to_dev(torch, p["v"]), core, pos0, n, p["max_ctx"], S)
    torch.cuda.synchronize()
    got = to_host(core).reshape(n, H, D)
    rows = np.arange(n)
    ref = O.prefill_f64(p["q"], p["qg"], S, p["k"], p["v"], pos0, p["max_ctx"], rows)
    st = O.compare(got, ref)
    report(f"prefill rescale pos0={pos0} n={n}", st)
    assert st["ok"], st


def test_ragged_late_max_moves(O, attn, torch_mod):
    lens = np.array([2500, 600, 9], np.uint32)
    r = O.ragged_inputs(77, lens)
    rng = np.random.default_rng(78)
    q_rows = r["q"].reshape(len(lens), H, D)
    k = r["k"].copy()
    for s, L in enumerate(lens):
        base = int(r["offsets"][s])
        for kvh in range(KV):
            for j, frac in enumerate((0.3, 0.7, 0.95)):
                sub = k[base:base + KV * int(L) * D]
                plant(sub, q_rows[s], kvh, int(L), int(frac * (int(L) - 1)), 8.0 + 9.0 * j, rng)
    r["k"] = k
    torch = torch_mod
    sc = attn.RaggedScratch(len(lens), int(lens.max()))
    core = torch.full((len(lens) * H * D,), -9123.5, device="cuda")
    attn.attn_decode_ragged(to_dev(torch, r["q"]), to_dev(torch, r["gate"]),
                            to_dev(torch, r["k"]), to_dev(torch, r["v"]),
                            to_dev(torch, r["offsets"]), to_dev(torch, r["lens"]), core, sc)
    torch.cuda.synchronize()
    got = to_host(core).reshape(len(lens), H, D)
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    st = O.compare(got, ref)
    report("ragged rescale", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st
