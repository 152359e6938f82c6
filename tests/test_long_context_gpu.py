"""The largest shapes the engine sizes for (a 262,144-token KV cache per layer,
src/engine/attention.hpp:35-41 and the survey's 5 GiB figure): decode over the whole cache, the
batched decode with a sequence far past its scratch's max_len, and a prefill chunk at a
128k-token prefix (sampled rows), each against the FP64 oracle."""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REF_REL_L2, report, to_dev, to_host

pytestmark = pytest.mark.gpu

H, KV, D = 16, 2, 256


@pytest.mark.parametrize("n_splits", [128, 60])
def test_decode_full_262k_cache(O, attn, torch_mod, n_splits):
    length = 262144
    d = O.decode_inputs(31, length, length, q_scale=1.0)
    torch = torch_mod
    core = torch.full((H * D,), -9123.5, device="cuda")
    sc = attn.DecodeScratch(n_splits)
    attn.attn_decode(to_dev(torch, d["q"]), to_dev(torch, d["qg"]), to_dev(torch, d["k"]),
                     to_dev(torch, d["v"]), core, sc, length, length, n_splits)
    torch.cuda.synchronize()
    got = to_host(core).reshape(H, D)
    ref = O.decode_f64(d["q"], d["qg"], d["k"], d["v"], length, length)
    st = O.compare(got, ref)
    report(f"decode len={length} splits={n_splits}", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st


def test_prefill_chunk_after_128k_prefix(O, attn, torch_mod):
    pos0, n = 131072, 48
    p = O.prefill_inputs(32, pos0, n, pos0 + n, q_scale=1.0)
    torch = torch_mod
    S = p["qg_stride"]
    core = torch.full((n * H * D,), -1.0, device="cuda")
    attn.attn_prefill(to_dev(torch, p["q"]), to_dev(torch, p["qg"]), to_dev(torch, p["k"]),
                      to_dev(torch, p["v"]), core, pos0, n, p["max_ctx"], S)
    torch.cuda.synchronize()
    got = to_host(core).reshape(n, H, D)
    rows = np.array([0, 1, 15, 16, 31, 32, 47])
    ref = O.prefill_f64(p["q"], p["qg"], S, p["k"], p["v"], pos0, p["max_ctx"], rows)
    st = O.compare(got[rows], ref)
    report(f"prefill pos0={pos0} n={n} rows={rows.size}", st)
    assert st["ok"], st


def test_ragged_sequence_far_past_max_len(O, attn, torch_mod):
    """max_len sizes the split slots for 512-key spans; a 65,536-key sequence then runs in
    spans 128x longer (every key is still attended)."""
    lens = np.array([65536, 700, 3], np.uint32)
    r = O.ragged_inputs(33, lens)
    torch = torch_mod
    sc = attn.RaggedScratch(len(lens), 512)
    core = torch.full((len(lens) * H * D,), -9123.5, device="cuda")
    attn.attn_decode_ragged(to_dev(torch, r["q"]), to_dev(torch, r["gate"]),
                            to_dev(torch, r["k"]), to_dev(torch, r["v"]),
                            to_dev(torch, r["offsets"]), to_dev(torch, r["lens"]), core, sc)
    torch.cuda.synchronize()
    got = to_host(core).reshape(len(lens), H, D)
    ref = O.ragged_f64(r["q"], r["gate"], r["k"], r["v"], r["offsets"], lens)
    st = O.compare(got, ref)
    report("ragged far past max_len", st)
    assert st["ok"], st
    assert st["rel_l2_head"] <= REF_REL_L2, st


def test_decode_fp8_full_262k_cache(O, attn, torch_mod):
    """The fp8 (e4m3 rows) decode over a whole 262,144-token cache, encoded on the GPU from the
    f16 cache, against the oracle on the same codes and scales."""
    length = 262144
    d = O.decode_inputs(33, length, length, q_scale=1.0)
    torch = torch_mod
    cache = attn.Fp8Cache(length)
    attn.attn_kv_encode_fp8(to_dev(torch, d["k"]), to_dev(torch, d["v"]), cache, 0, length)
    core = torch.full((H * D,), -9123.5, device="cuda")
    attn.attn_decode_fp8(to_dev(torch, d["q"]), to_dev(torch, d["qg"]), cache, core,
                         attn.DecodeScratch(128), length)
    torch.cuda.synchronize()
    got = to_host(core).reshape(H, D)
    k8, v8, ks, vs = (to_host(t) for t in cache.buffers())
    ref = O.decode_fp8_f64(d["q"], d["qg"], k8, v8, ks, vs, length, length)
    st = O.compare(got, ref)
    report(f"fp8 decode len={length}", st)
    assert st["ok"], st
