"""CPU tests of the C ABI boundary (include/miso_attn.h, miso_amd/lib/libmiso_attn.so): the
library loads without a GPU, exports exactly the declared entry points, validates arguments on
the host (no launch happens for a rejected call), and the split / grid policies keep their
contracts. No compute call is made here.
"""
from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "miso_attn.h"
EINVAL = 0x4D41


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(miso_attn_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from miso_amd import _lib
    return _lib.load()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 12
    for name in names:
        assert hasattr(lib, name), name
    from miso_amd import _lib
    assert sorted(_lib.SIGNATURES) == names  # the ctypes table matches the header
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r"\b(miso_attn_\w+)\b", out))
    assert exported == set(names)


def test_version_string(lib):
    assert lib.miso_attn_version().decode().startswith("miso_attn gfx950")


def rejected(rc, lib, needle):
    assert rc == EINVAL
    msg = lib.miso_attn_last_error().decode()
    assert needle in msg, msg


def test_host_validation_rejects_bad_arguments(lib):
    # P: a non-null, 16-byte aligned address that is never dereferenced -- every call below must
    # be rejected on the host before any launch.
    N, P = None, 0x10000
    rejected(lib.miso_attn_split(P, P, P, P, P, P, 0, 10, 1, N), lib, "len must be >= 1")
    rejected(lib.miso_attn_split(P, P, P, P, P, P, 11, 10, 1, N), lib, "exceeds max_ctx")
    rejected(lib.miso_attn_split(P, P, P, P, P, P, 5, 10, 0, N), lib, "n_splits")
    rejected(lib.miso_attn_combine(P, P, P, P, P, 0, N), lib, "n_splits")
    rejected(lib.miso_attn_decode(P, P, P, P, P, P, P, P, 0, 10, 4, N), lib, "len must be")
    # the allocation-free decode rejects split counts beyond its array before touching a device
    rejected(lib.miso_attn_decode_noalloc(P, P, P, P, P, 5, 10, 129, N), lib, "n_splits")
    rejected(lib.miso_attn_decode_noalloc(P, P, P, P, P, 5, 10, 0, N), lib, "n_splits")
    rejected(lib.miso_attn_decode_noalloc(P, P, P, P, P, 11, 10, 4, N), lib, "max_ctx")
    rejected(lib.miso_attn_prefill(P, P, P, P, P, 0, 0, 10, 8192, N), lib, "n must be >= 1")
    rejected(lib.miso_attn_prefill(P, P, P, P, P, 8, 3, 10, 8192, N), lib, "KV cache is full")
    rejected(lib.miso_attn_prefill(P, P, P, P, P, 0, 3, 10, 100, N), lib, "qg_stride")
    rejected(lib.miso_attn_prefill(P, P, P, P, P, 0, 3, 10, 8194, N), lib, "multiple of 4")
    W = 1 << 20
    rejected(lib.miso_attn_prefill_ws(P, P, P, P, P, 0, 0, 10, 8192, P, W, N), lib,
             "n must be >= 1")
    rejected(lib.miso_attn_prefill_ws(P, P, P, P, P, 8, 3, 10, 8192, P, W, N), lib,
             "KV cache is full")
    rejected(lib.miso_attn_prefill_ws(P, P, P, P, P, 0, 3, 10, 8192, N, W, N), lib, "workspace")
    rejected(lib.miso_attn_prefill_ws(P, P, P, P, P, 0, 3, 10, 8192, P + 4, W, N), lib,
             "workspace")
    need = lib.miso_attn_prefill_workspace_bytes(2000)
    rejected(lib.miso_attn_prefill_ws(P, P, P, P, P, 0, 2000, 2000, 8192, P, need - 1, N), lib,
             "smaller than")
    rejected(lib.miso_attn_prep(P, P, P, P, P, P, P, P, P, 10, 10, 1e-6, N), lib, "full")
    rejected(lib.miso_attn_prep_batch(P, P, P, P, P, P, P, P, P, 8, 10, 1e-6, 3, 9216, N), lib,
             "full")
    rejected(lib.miso_attn_prep_batch(P, P, P, P, P, P, P, P, P, 0, 10, 1e-6, 3, 8192, N), lib,
             "proj_stride")
    rejected(lib.miso_attn_decode_ragged(P, P, P, P, P, P, 0, 10, P, P, P, P, N), lib, "batch")
    rejected(lib.miso_attn_decode_ragged(P, P, P, P, P, P, 3, 0, P, P, P, P, N), lib, "max_len")
    paged = lib.miso_attn_decode_paged
    rejected(paged(P, P, P, P, P, 4, 16, P, 0, 10, P, P, P, P, N), lib, "batch")
    rejected(paged(P, P, P, P, P, 4, 16, P, 3, 0, P, P, P, P, N), lib, "max_len")
    rejected(paged(P, P, P, P, P, 0, 16, P, 3, 10, P, P, P, P, N), lib, "max_pages")
    for bad_page in (0, 4, 12, 131072):
        rejected(paged(P, P, P, P, P, 4, bad_page, P, 3, 10, P, P, P, P, N), lib, "page_size")
    rejected(paged(P, P, P, P, P, 4, 16, P, 3, 65, P, P, P, P, N), lib, "max_pages * page_size")
    enc, prep8, dec8 = lib.miso_attn_kv_encode_fp8, lib.miso_attn_prep_fp8, lib.miso_attn_decode_fp8
    rejected(enc(P, P, P, P, P, P, 8, 3, 10, N), lib, "max_ctx")
    rejected(prep8(P, P, P, P, P, P, P, P, P, P, P, 10, 10, 1e-6, N), lib, "full")
    rejected(dec8(P, P, P, P, P, P, P, P, P, P, 0, 10, 4, N), lib, "len must be")
    rejected(dec8(P, P, P, P, P, P, P, P, P, P, 11, 10, 4, N), lib, "exceeds max_ctx")
    rejected(dec8(P, P, P, P, P, P, P, P, P, P, 5, 10, 0, N), lib, "n_splits")
    q4k = lib.miso_attn_q4k_gemv
    for bad_k in (0, 256, 1024, 3072, 16384):
        rejected(q4k(P, P, P, 8, bad_k, 1, N), lib, "k must be")
    rejected(q4k(P, P, P, 8, 2048, 2, N), lib, "act_format")
    assert q4k(N, N, N, 0, 7, 9, N) == 0  # n_rows == 0: no-op
    for bad_k in (0, 256, 3072):
        rejected(lib.miso_attn_q6k_gemv(P, P, P, 8, bad_k, N), lib, "k must be")
    assert lib.miso_attn_q6k_gemv(N, N, N, 0, 7, N) == 0
    pair = lib.miso_attn_q4k_q6k_gemv_pair
    rejected(pair(P, 0, P, P, 5, P, P, N), lib, "row counts")
    rejected(pair(P, 5, P, P, 0, P, P, N), lib, "row counts")
    rejected(pair(P + 4, 5, P, P, 5, P, P, N), lib, "NULL or not 16-byte aligned")
    qkv = lib.miso_attn_qkv_gemv
    for nq, nk, nv in ((0, 5, 5), (5, 0, 5), (5, 5, 0)):
        rejected(qkv(P, nq, P, P, nk, P, P, nv, P, P, N), lib, "row counts")
    rejected(qkv(P, 5, P, P, 5, P, P + 4, 5, P, P, N), lib, "NULL or not 16-byte aligned")
    gin, gemm = lib.miso_attn_gemm_input, lib.miso_attn_gemm
    for bad_k in (0, 128, 2049):
        rejected(gin(P, P, P, bad_k, 4, N), lib, "multiple of 256")
        rejected(gemm(P, 0, P, P, P, bad_k, 8, 4, 8, N), lib, "multiple of 256")
    assert gin(N, N, N, 7, 0, N) == 0  # n_tok == 0: no-op
    assert gemm(N, 9, N, N, N, 7, 8, 0, 0, N) == 0 and gemm(N, 9, N, N, N, 7, 0, 4, 0, N) == 0
    rejected(gemm(P, 2, P, P, P, 2048, 8, 4, 8, N), lib, "format")
    rejected(gemm(P, 0, P, P, P, 2048, 8, 4, 7, N), lib, "ldy")
    rejected(gemm(P, 0, P, P + 4, P, 2048, 8, 4, 8, N), lib, "NULL or not 16-byte aligned")
    assert gemm(P, 1, P, N, P, 2048, 8, 0, 8, N) == 0
    rejected(lib.miso_attn_combine_variant(7, P, P, P, P, P, 4, 0, 0, 0, N), lib, "variant")
    rejected(lib.miso_attn_combine_variant(0, P, P, P, P, P, 4, 0, 8, 2, N), lib, "range form")
    rejected(lib.miso_attn_combine_variant(1, P, P, P, P, P, 4, 60, 8, 2, N), lib, "range form")


def test_host_validation_rejects_null_and_misaligned_pointers(lib):
    N, P = None, 0x10000
    bad = "NULL or not 16-byte aligned"
    for q in (N, P + 4, P + 8):
        rejected(lib.miso_attn_split(q, P, P, P, P, P, 5, 10, 1, N), lib, bad)
        rejected(lib.miso_attn_prefill(P, P, q, P, P, 0, 3, 10, 8192, N), lib, bad)
        rejected(lib.miso_attn_combine(P, P, P, P, q, 4, N), lib, bad)
        rejected(lib.miso_attn_decode(P, P, P, P, P, P, P, q, 5, 10, 4, N), lib, bad)
        rejected(lib.miso_attn_prep(P, P, P, P, P, P, q, P, P, 1, 10, 1e-6, N), lib, bad)
        rejected(lib.miso_attn_prep_batch(P, P, P, P, P, P, P, P, q, 0, 10, 1e-6, 3, 9216, N),
                 lib, bad)
        rejected(lib.miso_attn_decode_ragged(P, P, q, P, P, P, 3, 10, P, P, P, P, N), lib, bad)
        rejected(lib.miso_attn_combine_variant(3, P, P, q, P, P, 4, 0, 0, 0, N), lib, bad)
    # part_m / part_l are scalar arrays: 4-byte alignment suffices, NULL and odd addresses do not
    rejected(lib.miso_attn_split(P, P, P, N, P, P, 5, 10, 1, N), lib, bad)
    rejected(lib.miso_attn_combine(P, P + 2, P, P, P, 4, N), lib, bad)
    rejected(lib.miso_attn_decode_ragged(P, P, P, P, N, P, 3, 10, P, P, P, P, N), lib, bad)
    for q in (N, P + 4):
        rejected(lib.miso_attn_decode_paged(P, P, q, P, P, 4, 16, P, 3, 10, P, P, P, P, N), lib,
                 bad)
    rejected(lib.miso_attn_decode_paged(P, P, P, P, N, 4, 16, P, 3, 10, P, P, P, P, N), lib, bad)
    rejected(lib.miso_attn_decode_paged(P, P, P, P, P, 4, 16, N, 3, 10, P, P, P, P, N), lib, bad)
    # fp8 cache: codes need 16-byte alignment, the per-row scales 4-byte alignment
    for q in (N, P + 4):
        rejected(lib.miso_attn_kv_encode_fp8(P, P, q, P, P, P, 0, 3, 10, N), lib, bad)
        rejected(lib.miso_attn_prep_fp8(P, P, P, P, P, P, P, q, P, P, P, 1, 10, 1e-6, N), lib,
                 bad)
        rejected(lib.miso_attn_decode_fp8(P, P, q, P, P, P, P, P, P, P, 5, 10, 4, N), lib, bad)
    for s_bad in (N, P + 2):
        rejected(lib.miso_attn_kv_encode_fp8(P, P, P, P, s_bad, P, 0, 3, 10, N), lib, bad)
        rejected(lib.miso_attn_prep_fp8(P, P, P, P, P, P, P, P, P, s_bad, P, 1, 10, 1e-6, N),
                 lib, bad)
        rejected(lib.miso_attn_decode_fp8(P, P, P, P, s_bad, P, P, P, P, P, 5, 10, 4, N), lib,
                 bad)
    assert lib.miso_attn_kv_encode_fp8(N, N, N, N, N, N, 0, 0, 10, N) == 0  # n == 0: no-op
    for q in (N, P + 4):
        rejected(lib.miso_attn_q4k_gemv(q, P, P, 8, 2048, 1, N), lib, bad)
        rejected(lib.miso_attn_q4k_gemv(P, q, P, 8, 2048, 1, N), lib, bad)
    rejected(lib.miso_attn_q4k_gemv(P, P, P + 2, 8, 2048, 1, N), lib, bad)
    for q in (N, P + 4):
        rejected(lib.miso_attn_q6k_gemv(q, P, P, 8, 2048, N), lib, bad)


def test_python_layer_raises_runtime_error_with_message():
    from miso_amd import _lib
    with pytest.raises(RuntimeError, match="n_splits must be >= 1"):
        P = 0x10000
        _lib.check(_lib.load().miso_attn_combine(P, P, P, P, P, 0, None))


def test_split_policy_contract(lib):
    f = lib.miso_attn_n_splits
    assert f(0, 60) == 1 and f(0, 0) == 1 and f(5, 0) == 1
    prev = 1
    for length in list(range(1, 3000, 7)) + [32767, 32768, 32769, 10**6]:
        for cap in (1, 3, 16, 60, 128, 256):
            n = f(length, cap)
            assert 1 <= n <= cap and n <= 128
            assert n <= (length + 31) // 32
        n60 = f(length, 60)
        assert n60 >= prev or length < 32  # non-decreasing in length
        prev = n60
    assert f(32768, 60) == 60 and f(32768, 1000) == 128 and f(512, 60) == 16


def test_prefill_grid_covers_every_block(lib):
    for n in (1, 15, 16, 17, 31, 32, 33, 63, 64, 65, 2048, 4095, 4096, 8192, 10**5):
        items = lib.miso_attn_prefill_items(n)
        tokens = 32 if n >= 4096 else 16  # tokens per workgroup (two row blocks per wave from 4096)
        blocks = (n + tokens - 1) // tokens
        assert items % 8 == 0 and items >= 2 * blocks and items < 2 * blocks + 8
        # item -> (kv head, rank): a bijection onto {0,1} x [0, blocks) plus idle slots
        seen = set()
        for item in range(items):
            slot = item % 8
            rank = (item // 8) * 4 + slot % 4
            if rank < blocks:
                seen.add((slot // 4, rank))
        assert len(seen) == 2 * blocks


def test_ragged_scratch_sizes(lib):
    assert lib.miso_attn_ragged_splits(1) == 1
    assert lib.miso_attn_ragged_splits(512) == 1 and lib.miso_attn_ragged_splits(513) == 2
    assert lib.miso_attn_ragged_splits(16384) == 32
    assert lib.miso_attn_ragged_partials(64, 16384) == 64 * 2 * 32 * 8


def test_prefill_workspace_bytes(lib):
    """The balanced prefill's workspace (n <= 2048, 3841 <= n <= 4096): a fixed 1 KiB of pair
    counters, then (m, l) and O of both parts of each pair (128 rows per part with 16-token
    blocks up to 2048 tokens, 256 with 32-token blocks above); nothing for the launches that take
    the plain layout."""
    for n in (0, 2049, 3000, 3840, 4097, 8192, 1 << 20):
        assert lib.miso_attn_prefill_workspace_bytes(n) == 0
    for n in (1, 16, 17, 32, 33, 1000, 2047, 2048, 3841, 4000, 4095, 4096):
        tokens = 16 if n <= 2048 else 32
        pairs = 2 * (((n + tokens - 1) // tokens) // 2)
        rows = 8 * tokens
        assert lib.miso_attn_prefill_workspace_bytes(n) == 1024 + pairs * 2 * rows * 258 * 4
    assert max(lib.miso_attn_prefill_workspace_bytes(n) for n in range(1, 4200, 7)) == \
        lib.miso_attn_prefill_workspace_bytes(4096)


def test_layer_core_offsets(lib):
    """The engine's scratch.core / ps.core inside the layer workspaces: 16-byte aligned, inside
    the workspace, and not overlapping the balanced prefill's counters at the prefill workspace's
    end."""
    dec = lib.miso_attn_layer_decode_core()
    assert dec % 4 == 0 and dec + 4096 <= lib.miso_attn_layer_decode_ws()
    for max_tok in (1, 16, 512, 4096, 8192):
        at = lib.miso_attn_layer_prefill_core(max_tok)
        balance = lib.miso_attn_prefill_workspace_bytes(min(max_tok, 4096)) // 4
        assert at % 4 == 0
        assert at + max_tok * 4096 <= lib.miso_attn_layer_prefill_ws(max_tok) - balance
