"""Paged batched decode (no reference counterpart): the ragged decode's keys scattered over a pool
of KV pages in a random order must give bit-identical outputs to the contiguous ragged path
(same splits, same arithmetic), and so the same parity against the FP64 oracle."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REF_REL_L2, report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, KV, D = 16, 2, 256


def paginate(r, lens, page, seed, spare=3):
    """Pool of pages in a random order holding each sequence's K/V [2][len][256]; page g is
    [2][page][256]. Returns (k_pages, v_pages, table [batch][max_pages]); unused table entries
    and rows past a sequence's end point at valid pages (never read)."""
    lens = np.asarray(lens, np.int64)
    npg = (lens + page - 1) // page
    max_pages = max(1, int(npg.max()))
    total = int(npg.sum()) + spare
    perm = np.random.default_rng(seed).permutation(total).astype(np.int32)
    kp = np.random.default_rng(seed + 1).integers(0, 0x3C00, (total, KV, page, D), dtype=np.uint16)
    vp = kp.copy()
    table = np.zeros((len(lens), max_pages), np.int32)
    nxt = 0
    for s, L in enumerate(lens):
        o = int(r["offsets"][s])
        k = r["k"][o:o + KV * L * D].reshape(KV, L, D)
        v = r["v"][o:o + KV * L * D].reshape(KV, L, D)
        for j in range(int(npg[s])):
            g = int(perm[nxt])
            nxt += 1
            table[s, j] = g
            rows = min(page, L - j * page)
            kp[g, :, :rows] = k[:, j * page:j * page + rows]
            vp[g, :, :rows] = v[:, j * page:j * page + rows]
    return kp.reshape(-1), vp.reshape(-1), table


def run_both(O, attn, torch, lens, seed, page, max_len=None):
    r = O.ragged_inputs(seed, lens)
    batch = len(lens)
    max_len = int(max(lens)) if max_len is None else max_len
    sc = attn.RaggedScratch(batch, max_len)
    q, gate = to_dev(torch, r["q"]), to_dev(torch, r["gate"])
    d_lens = to_dev(torch, r["lens"])
    ragged = torch.full((batch * H * D,), -9123.5, device="cuda")
    attn.attn_decode_ragged(q, gate, to_dev(torch, r["k"]), to_dev(torch, r["v"]),
                            to_dev(torch, r["offsets"]), d_lens, ragged, sc)
    kp, vp, table = paginate(r, lens, page, seed)
    paged = torch.full((batch * H * D,), 7777.25, device="cuda")
    attn.attn_decode_paged(q, gate, to_dev(torch, kp), to_dev(torch, vp),
                           torch.from_numpy(table).cuda(), page, d_lens, paged, sc)
    torch.cuda.synchronize()
    return r, to_host(ragged).reshape(batch, H, D), to_host(paged).reshape(batch, H, D)


@pytest.mark.parametrize("page", [8, 16, 64, 256])
def test_paged_bit_identical_to_ragged(O, attn, torch_mod, page):
    """Lengths at unit, page and split boundaries, a single key, and longer sequences."""
    lens = np.array([1, 7, 8, 9, 15, 16, 17, 63, 64, 65, 511, 512, 513, 1500, 3000], np.uint32)
    _, ragged, paged = run_both(O, attn, torch_mod, lens, 11 + page, page)
    assert np.array_equal(ragged.view(np.uint32), paged.view(np.uint32))


def test_paged_long_spans_read_table_beyond_lane_slice(O, attn, torch_mod):
    """max_len below the true maximum: a 2049-key sequence in 2 spans of ~1024 keys, i.e. 128
    pages of 8 rows per span (the slice held in lanes covers 64)."""
    lens = np.array([2049, 300, 5], np.uint32)
    r, ragged, paged = run_both(O, attn, torch_mod, lens, 21, 8, max_len=600)
    assert np.array_equal(ragged.view(np.uint32), paged.view(np.uint32))
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    st = O.compare(paged, ref)
    report("paged long spans", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st


def test_paged_c5_shape(O, attn, torch_mod):
    """C5's length distribution (64 sequences, U[1024, 16384], seed 64) with 16-row pages: the
    same outputs as the ragged path, which test_ragged_c5 checks against the oracle."""
    lens = O.ragged_lengths(64, 64, 1024, 16384)
    _, ragged, paged = run_both(O, attn, torch_mod, lens, 64, 16)
    assert np.array_equal(ragged.view(np.uint32), paged.view(np.uint32))


def test_paged_wide_batch_fallback(O, attn, torch_mod):
    """600 sequences, above the streaming kernels' batch limit: both layouts run one workgroup
    per (sequence, KV head, split) slot, still bit-identical."""
    lens = np.random.default_rng(601).integers(0, 700, 600).astype(np.uint32)
    _, ragged, paged = run_both(O, attn, torch_mod, lens, 601, 16)
    assert np.array_equal(ragged.view(np.uint32), paged.view(np.uint32))


def test_paged_empty_sequence_is_zero(O, attn, torch_mod):
    lens = np.array([5, 0, 9], np.uint32)
    _, ragged, paged = run_both(O, attn, torch_mod, lens, 6, 8, max_len=16)
    assert not paged[1].any()
    assert np.array_equal(ragged.view(np.uint32), paged.view(np.uint32))


def test_paged_lens_past_the_table_are_clamped(O, attn, torch_mod):
    """lens[s] above max_pages * page_size: the sequence attends to the keys its page-table row
    addresses (the first max_pages pages), in the split and in the merge, i.e. exactly the ragged
    decode of the clamped lengths. The table's allocation continues with valid page ids past its
    last row, so a read beyond a row would show as different values, not as a fault."""
    torch = torch_mod
    page, max_pages = 8, 4
    cap = page * max_pages
    lens = np.array([40, 100, 7, 33], np.uint32)
    cut = np.minimum(lens, cap).astype(np.uint32)
    batch = len(lens)
    r = O.ragged_inputs(31, cut)
    sc = attn.RaggedScratch(batch, cap)
    q, gate = to_dev(torch, r["q"]), to_dev(torch, r["gate"])
    ragged = torch.full((batch * H * D,), -9123.5, device="cuda")
    attn.attn_decode_ragged(q, gate, to_dev(torch, r["k"]), to_dev(torch, r["v"]),
                            to_dev(torch, r["offsets"]), to_dev(torch, cut), ragged, sc)
    kp, vp, table = paginate(r, cut, page, 31)
    assert table.shape == (batch, max_pages)
    padded = torch.zeros((batch + 16, max_pages), dtype=torch.int32, device="cuda")
    padded[:batch] = torch.from_numpy(table).cuda()
    paged = torch.full((batch * H * D,), 7777.25, device="cuda")
    attn.attn_decode_paged(q, gate, to_dev(torch, kp), to_dev(torch, vp), padded[:batch], page,
                           to_dev(torch, lens), paged, sc)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(ragged).view(np.uint32), to_host(paged).view(np.uint32))
