"""Ragged batched decode parity (BASELINE C5; no reference counterpart -- the reference is
batch-1): each sequence against the FP64 oracle of decode with a dense sigmoid gate.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REF_REL_L2, report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, D = 16, 256


def run(O, attn, torch, lens, seed, max_len=None):
    r = O.ragged_inputs(seed, lens)
    batch = len(lens)
    max_len = int(max(lens)) if max_len is None else max_len
    sc = attn.RaggedScratch(batch, max_len)
    core = torch.full((batch * H * D,), -9123.5, device="cuda")
    attn.attn_decode_ragged(to_dev(torch, r["q"]), to_dev(torch, r["gate"]),
                            to_dev(torch, r["k"]), to_dev(torch, r["v"]),
                            to_dev(torch, r["offsets"]), to_dev(torch, r["lens"]), core, sc)
    torch.cuda.synchronize()
    return r, to_host(core).reshape(batch, H, D)


def test_ragged_c5(O, attn, torch_mod):
    """C5: 64 sequences, lengths uniform in [1024, 16384] from seed 64."""
    lens = O.ragged_lengths(64, 64, 1024, 16384)
    r, got = run(O, attn, torch_mod, lens, 64)
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    st = O.compare(got, ref)
    report(f"C5 sum_len={int(lens.sum())}", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st


def test_ragged_edges(O, attn, torch_mod):
    """Lengths at and around the span unit and chunk boundaries, a single-key sequence, and a
    max_len below the true maximum (spans grow instead of keys being dropped)."""
    lens = np.array([1, 7, 8, 9, 511, 512, 513, 2049, 3], np.uint32)
    for max_len in (None, 600):
        r, got = run(O, attn, torch_mod, lens, 5, max_len)
        ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
        st = O.compare(got, ref)
        assert st["ok"], (max_len, st)
        assert st["rel_l2_head"] <= REF_REL_L2, (max_len, st)


def test_ragged_empty_sequence_is_zero(O, attn, torch_mod):
    lens = np.array([5, 0, 9], np.uint32)
    r, got = run(O, attn, torch_mod, lens, 6, 16)
    assert not got[1].any()
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"],
                       np.array([5, 1, 9], np.uint32))
    for s in (0, 2):
        assert O.compare(got[s], ref[s])["ok"]


def check_all(O, attn, torch, lens, seed, max_len=None, name="ragged"):
    r, got = run(O, attn, torch, lens, seed, max_len)
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    live = np.asarray(lens) > 0
    st = O.compare(got[live], ref[live])
    report(f"{name} batch={len(lens)} sum_len={int(np.sum(lens))}", st)
    assert st["ok"] and st["rel_l2_head"] <= REF_REL_L2, st
    assert not got[~live].any()


def test_ragged_stream_many_short_items(O, attn, torch_mod):
    """The streaming split (one workgroup per CU, each wave's tile stream running across items)
    over many items of one or two 32-key tiles -- most waves have no tile in most items, and the
    query rows alternate between the two LDS slots at every item -- with empty sequences among
    them and a few long ones."""
    rng = np.random.default_rng(300)
    lens = rng.integers(1, 65, 300).astype(np.uint32)
    lens[::37] = 0
    lens[[5, 150, 299]] = (3000, 1025, 513)
    check_all(O, attn, torch_mod, lens, 300, name="stream short items")


def test_ragged_stream_empty_span(O, attn, torch_mod):
    """A sequence longer than max_len: its split count is capped at max_len's, and with 65537
    keys in 128 splits of 65 units the last split's span is empty (its partial is written as
    (-inf, 0, 0) without tiles)."""
    lens = np.array([65537, 700, 33], np.uint32)
    check_all(O, attn, torch_mod, lens, 65537, max_len=65536, name="stream empty span")


def test_ragged_wide_batch_fallback(O, attn, torch_mod):
    """A batch above the streaming split's descriptor limit (512 sequences) runs one workgroup
    per (sequence, KV head, split); same gates."""
    rng = np.random.default_rng(600)
    lens = rng.integers(0, 700, 600).astype(np.uint32)
    check_all(O, attn, torch_mod, lens, 600, name="fallback batch")


def test_ragged_stream_equals_split_kernel(O, attn, torch_mod):
    """The streaming kernel and the one-workgroup-per-split kernel compute each item the same
    way: a 600-sequence batch (above the streaming limit of 512) and its first 100 sequences as
    a batch of their own (streamed) give bit-identical rows. Both run with max_len 6144, so both
    launches split at the wide chunk."""
    torch = torch_mod
    rng = np.random.default_rng(602)
    lens = rng.integers(0, 1100, 600).astype(np.uint32)
    r = O.ragged_inputs(602, lens)
    q, gate = to_dev(torch, r["q"]), to_dev(torch, r["gate"])
    k, v = to_dev(torch, r["k"]), to_dev(torch, r["v"])
    offs, d_lens = to_dev(torch, r["offsets"]), to_dev(torch, r["lens"])
    out = {}
    for batch in (600, 100):
        assert attn.ragged_chunk(batch, 6144) == 1024
        sc = attn.RaggedScratch(batch, 6144)
        core = torch.full((batch * H * D,), -9123.5, device="cuda")
        attn.attn_decode_ragged(q[:batch * H * D], gate[:batch * H * D], k, v, offs[:batch],
                                d_lens[:batch], core, sc)
        torch.cuda.synchronize()
        out[batch] = to_host(core).reshape(batch, H, D)
    assert np.array_equal(out[600][:100].view(np.uint32), out[100].view(np.uint32))


def test_ragged_chunk_policy(attn, torch_mod):
    """Spans of 1024 keys once they still give four per CU, else 512: C5 (64 sequences up to
    16384 keys) takes the wide chunk, a single 64k-key sequence or a small batch the narrow one."""
    cus = torch_mod.cuda.get_device_properties(0).multi_processor_count
    assert attn.ragged_chunk(64, 16384) == (1024 if 2 * 64 * 16 >= 4 * cus else 512)
    assert attn.ragged_chunk(1, 65536) == 512
    assert attn.ragged_chunk(9, 2049) == 512
