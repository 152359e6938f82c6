"""The allocation-free decode entry point (miso_attn_decode_noalloc) against miso_attn_decode,
through the C ABI: bit-identical outputs on two calls in a row, the second with fewer keys and
splits (the library's device array keeps the first call's partials; the second must not read
them), then the first size again.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import to_dev, to_host

pytestmark = pytest.mark.gpu

H, D = 16, 256


def decode_pair(O, attn, torch, length, max_splits, seed):
    from miso_amd import _lib
    lib = _lib.load()
    d = O.decode_inputs(seed, length, length + 5, q_scale=2.0)
    q, qg = to_dev(torch, d["q"]), to_dev(torch, d["qg"])
    k, v = to_dev(torch, d["k"]), to_dev(torch, d["v"])
    n = attn.attn_n_splits(length, max_splits)
    ref = torch.full((H * D,), -9123.5, device="cuda")
    attn.attn_decode(q, qg, k, v, ref, attn.DecodeScratch(max_splits), length, d["max_ctx"], n)
    got = torch.full((H * D,), -9123.5, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.miso_attn_decode_noalloc(q.data_ptr(), qg.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      got.data_ptr(), length, d["max_ctx"], n, stream)
    _lib.check(rc)
    torch.cuda.synchronize()
    return d, to_host(got), to_host(ref), n


def test_noalloc_decode_matches_decode_on_consecutive_calls(O, attn, torch_mod):
    for length, cap, seed in ((32768, 128, 41), (1000, 128, 42), (4099, 60, 43), (32768, 128, 44)):
        d, got, ref, n = decode_pair(O, attn, torch_mod, length, cap, seed)
        print(f"[noalloc] len={length} splits={n}", flush=True)
        assert not (got == -9123.5).any()
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), (length, n)
        st = O.compare(got.reshape(H, D),
                       O.decode_f64(d["q"], d["qg"], d["k"], d["v"], length, d["max_ctx"]))
        assert st["ok"] and st["rel_l2_head"] <= 1e-5, st


def test_noalloc_decode_rejects_too_many_splits(attn, torch_mod):
    from miso_amd import _lib
    lib = _lib.load()
    t = torch_mod.zeros(16, device="cuda")
    p = t.data_ptr()
    rc = lib.miso_attn_decode_noalloc(p, p, p, p, p, 5000, 5000, 129, None)
    assert rc == 0x4D41 and b"n_splits" in lib.miso_attn_last_error()
