"""Host-side operators over torch device tensors, calling the C ABI of libmiso_attn.so.

The names and argument meanings mirror the reference's kernel launch sites (kernels/
attention_decode.hpp, kernels/attention_prefill.hpp as launched by src/engine/attention.hip and
tests/test_attn_splitk.hip): the caller owns every buffer, including the split partials, and
calls only enqueue work on the given stream (default: torch's current stream). Failures raise
RuntimeError, as the reference throws std::runtime_error.

torch is used for device memory and streams only; all arithmetic runs in the HIP kernels.
"""
from __future__ import annotations

import ctypes
from typing import Optional

import torch

from . import _lib

Q_HEADS, KV_HEADS, DIM, GROUP = 16, 2, 256, 8
QG_STRIDE = Q_HEADS * 2 * DIM  # 8192: [16][512] (q half, gate half) per token


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream(stream) -> Optional[int]:
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else int(stream)


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, numel: int) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.numel() < numel:
        raise ValueError(f"{name} has {t.numel()} elements, needs >= {numel}")


def _cache_dtype(t: torch.Tensor) -> torch.dtype:
    return torch.float16 if t.dtype == torch.float16 else torch.int16


def attn_n_splits(length: int, max_splits: int) -> int:
    """Split count for a decode over `length` keys with partial buffers for max_splits splits."""
    return int(_lib.load().miso_attn_n_splits(length, max_splits))


def attn_prefill_items(n: int) -> int:
    return int(_lib.load().miso_attn_prefill_items(n))


def attn_prep(qg, k, v, q_norm, k_norm, inv_freq, k_cache, v_cache, q, pos: int, max_ctx: int,
              eps: float, stream=None) -> None:
    """RMSNorm + RoPE of one token's 16 query and 2 key heads; appends K/V at `pos`."""
    f32 = torch.float32
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(k, "k", f32, KV_HEADS * DIM)
    _need(v, "v", f32, KV_HEADS * DIM)
    _need(q_norm, "q_norm", f32, DIM)
    _need(k_norm, "k_norm", f32, DIM)
    _need(inv_freq, "inv_freq", f32, 32)
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * max_ctx * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * max_ctx * DIM)
    _need(q, "q", f32, Q_HEADS * DIM)
    _lib.check(_lib.load().miso_attn_prep(
        _ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(inv_freq), _ptr(k_cache),
        _ptr(v_cache), _ptr(q), pos, max_ctx, eps, _stream(stream)))


def attn_prep_batch(qg, k, v, q_norm, k_norm, inv_freq, k_cache, v_cache, q, pos0: int,
                    max_ctx: int, eps: float, n: int, proj_stride: int, stream=None) -> None:
    """attn_prep for n tokens; qg/k/v are views into a token-major projection buffer whose
    rows are proj_stride floats apart."""
    f32 = torch.float32
    for name, t in (("qg", qg), ("k", k), ("v", v)):
        if not t.is_cuda or t.dtype != f32:
            raise ValueError(f"{name} must be a float32 device tensor")
    _need(q_norm, "q_norm", f32, DIM)
    _need(k_norm, "k_norm", f32, DIM)
    _need(inv_freq, "inv_freq", f32, 32)
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * max_ctx * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * max_ctx * DIM)
    _need(q, "q", f32, n * Q_HEADS * DIM)
    _lib.check(_lib.load().miso_attn_prep_batch(
        _ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(inv_freq), _ptr(k_cache),
        _ptr(v_cache), _ptr(q), pos0, max_ctx, eps, n, proj_stride, _stream(stream)))


def attn_split(q, k_cache, v_cache, part_m, part_l, part_o, length: int, max_ctx: int,
               n_splits: int, stream=None, valu: bool = False) -> None:
    """Split-K partials (miso_attn_split; with valu, the VALU form miso_attn_split_valu)."""
    f32 = torch.float32
    _need(q, "q", f32, Q_HEADS * DIM)
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * max_ctx * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * max_ctx * DIM)
    _need(part_m, "part_m", f32, KV_HEADS * n_splits * GROUP)
    _need(part_l, "part_l", f32, KV_HEADS * n_splits * GROUP)
    _need(part_o, "part_o", f32, KV_HEADS * n_splits * GROUP * DIM)
    lib = _lib.load()
    fn = lib.miso_attn_split_valu if valu else lib.miso_attn_split
    _lib.check(fn(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(part_m), _ptr(part_l), _ptr(part_o), length,
        max_ctx, n_splits, _stream(stream)))


def attn_combine(part_m, part_l, part_o, qg, core, n_splits: int, stream=None) -> None:
    f32 = torch.float32
    _need(part_m, "part_m", f32, KV_HEADS * n_splits * GROUP)
    _need(part_l, "part_l", f32, KV_HEADS * n_splits * GROUP)
    _need(part_o, "part_o", f32, KV_HEADS * n_splits * GROUP * DIM)
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(core, "core", f32, Q_HEADS * DIM)
    _lib.check(_lib.load().miso_attn_combine(
        _ptr(part_m), _ptr(part_l), _ptr(part_o), _ptr(qg), _ptr(core), n_splits,
        _stream(stream)))


def attn_combine_variant(variant: int, part_m, part_l, part_o, qg, core, n_splits: int,
                         first: int = 0, count: int = 0, grid: int = 0, stream=None) -> None:
    """The header API's combine template variants (0: <256>, 1: <64>, 2: <64,true>,
    3: <64,true,4>) with the reference's launch shapes, or with count > 0 the range form
    attn_combine_op<64,...>(p, first, count) on `grid` 64-thread workgroups."""
    f32 = torch.float32
    _need(part_m, "part_m", f32, KV_HEADS * n_splits * GROUP)
    _need(part_l, "part_l", f32, KV_HEADS * n_splits * GROUP)
    _need(part_o, "part_o", f32, KV_HEADS * n_splits * GROUP * DIM)
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(core, "core", f32, Q_HEADS * DIM)
    _lib.check(_lib.load().miso_attn_combine_variant(
        variant, _ptr(part_m), _ptr(part_l), _ptr(part_o), _ptr(qg), _ptr(core), n_splits, first,
        count, grid, _stream(stream)))


class DecodeScratch:
    """Caller-owned split partials with capacity for max_splits splits (the role of
    AttentionScratch::part_m/part_l/part_o in the reference engine)."""

    def __init__(self, max_splits: int, device="cuda"):
        self.max_splits = max_splits
        n = KV_HEADS * max_splits * GROUP
        self.part_m = torch.empty(n, dtype=torch.float32, device=device)
        self.part_l = torch.empty(n, dtype=torch.float32, device=device)
        self.part_o = torch.empty(n * DIM, dtype=torch.float32, device=device)
        # the single-launch decode's arrival counters (zero; every call leaves them zero)
        self.sync = torch.zeros(4, dtype=torch.int32, device=device)


def attn_decode(q, qg, k_cache, v_cache, core, scratch: DecodeScratch, length: int,
                max_ctx: int, n_splits: Optional[int] = None, stream=None,
                f16_query: bool = False, fused: bool = False) -> int:
    """Split + combine for one decode token over keys [0, length), in the reference's f32
    arithmetic (or, with f16_query, the f16-query / f16-numerator variant
    miso_attn_decode_f16q; with fused, both in one launch, miso_attn_decode_fused). Returns
    n_splits used."""
    if n_splits is None:
        n_splits = attn_n_splits(length, scratch.max_splits)
    if n_splits > scratch.max_splits:
        raise ValueError("n_splits exceeds the scratch capacity")
    f32 = torch.float32
    _need(q, "q", f32, Q_HEADS * DIM)
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * max_ctx * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * max_ctx * DIM)
    _need(core, "core", f32, Q_HEADS * DIM)
    lib = _lib.load()
    if fused:
        if f16_query:
            raise ValueError("the single-launch decode computes in the reference's f32 arithmetic")
        _lib.check(lib.miso_attn_decode_fused(
            _ptr(q), _ptr(qg), _ptr(k_cache), _ptr(v_cache), _ptr(core), _ptr(scratch.part_m),
            _ptr(scratch.part_l), _ptr(scratch.part_o), _ptr(scratch.sync), length, max_ctx,
            n_splits, _stream(stream)))
        return n_splits
    fn = lib.miso_attn_decode_f16q if f16_query else lib.miso_attn_decode
    _lib.check(fn(
        _ptr(q), _ptr(qg), _ptr(k_cache), _ptr(v_cache), _ptr(core), _ptr(scratch.part_m),
        _ptr(scratch.part_l), _ptr(scratch.part_o), length, max_ctx, n_splits, _stream(stream)))
    return n_splits


def prefill_workspace_bytes(n: int) -> int:
    return int(_lib.load().miso_attn_prefill_workspace_bytes(n))


class PrefillScratch:
    """Workspace of the balanced prefill (miso_attn_prefill_ws) for launches of up to max_n
    tokens (the form covers n <= 2048 and 3841 <= n <= 4096), zero-filled once; every call leaves
    it reusable."""

    def __init__(self, max_n: int = 4096, device="cuda"):
        nbytes = max(prefill_workspace_bytes(min(max_n, 2048)),
                     prefill_workspace_bytes(min(max_n, 4096)))
        self.buf = torch.zeros(max((nbytes + 3) // 4, 4), dtype=torch.int32, device=device)
        self.nbytes = self.buf.numel() * 4


def attn_prefill(q, qg, k_cache, v_cache, core, pos0: int, n: int, max_ctx: int,
                 qg_stride: int = QG_STRIDE, stream=None, scratch: PrefillScratch = None) -> None:
    """Causal prefill of tokens pos0 .. pos0 + n - 1; with `scratch`, the balanced form
    (miso_attn_prefill_ws)."""
    f32 = torch.float32
    _need(q, "q", f32, n * Q_HEADS * DIM)
    _need(qg, "qg", f32, (n - 1) * qg_stride + Q_HEADS * 2 * DIM if n else 0)
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * max_ctx * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * max_ctx * DIM)
    _need(core, "core", f32, n * Q_HEADS * DIM)
    if scratch is None:
        _lib.check(_lib.load().miso_attn_prefill(
            _ptr(q), _ptr(qg), _ptr(k_cache), _ptr(v_cache), _ptr(core), pos0, n, max_ctx,
            qg_stride, _stream(stream)))
    else:
        _lib.check(_lib.load().miso_attn_prefill_ws(
            _ptr(q), _ptr(qg), _ptr(k_cache), _ptr(v_cache), _ptr(core), pos0, n, max_ctx,
            qg_stride, _ptr(scratch.buf), scratch.nbytes, _stream(stream)))


def ragged_partials(batch: int, max_len: int) -> int:
    return int(_lib.load().miso_attn_ragged_partials(batch, max_len))


def ragged_chunk(batch: int, max_len: int) -> int:
    """Keys per span the ragged / paged decode of such a batch uses on the current device."""
    return int(_lib.load().miso_attn_ragged_chunk(batch, max_len))


class RaggedScratch:
    def __init__(self, batch: int, max_len: int, device="cuda"):
        n = ragged_partials(batch, max_len)
        self.batch, self.max_len = batch, max_len
        self.part_m = torch.empty(n, dtype=torch.float32, device=device)
        self.part_l = torch.empty(n, dtype=torch.float32, device=device)
        self.part_o = torch.empty(n * DIM, dtype=torch.float32, device=device)


def attn_decode_ragged(q, gate, k_cache, v_cache, kv_offsets, lens, core,
                       scratch: RaggedScratch, stream=None) -> None:
    """Batched decode: sequence s attends over lens[s] keys stored as K/V [2][lens[s]][256]
    starting kv_offsets[s] halves into k_cache / v_cache (device int64 / int32 arrays)."""
    batch, max_len = scratch.batch, scratch.max_len
    f32 = torch.float32
    _need(q, "q", f32, batch * Q_HEADS * DIM)
    _need(gate, "gate", f32, batch * Q_HEADS * DIM)
    _need(core, "core", f32, batch * Q_HEADS * DIM)
    _need(kv_offsets, "kv_offsets", torch.int64, batch)
    _need(lens, "lens", torch.int32, batch)
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        if not t.is_cuda or t.dtype not in (torch.float16, torch.int16):
            raise ValueError(f"{name} must be a float16 device tensor")
    _lib.check(_lib.load().miso_attn_decode_ragged(
        _ptr(q), _ptr(gate), _ptr(k_cache), _ptr(v_cache), _ptr(kv_offsets), _ptr(lens), batch,
        max_len, _ptr(core), _ptr(scratch.part_m), _ptr(scratch.part_l), _ptr(scratch.part_o),
        _stream(stream)))


def attn_decode_paged(q, gate, k_pages, v_pages, page_table, page_size: int, lens, core,
                      scratch: RaggedScratch, stream=None) -> None:
    """Batched decode over a KV page pool: page g holds [2][page_size][256] f16 at
    g * 2 * page_size * 256 of k_pages / v_pages; sequence s's positions
    [j * page_size, (j + 1) * page_size) are in page page_table[s, j] (device int32
    [batch][max_pages]). Same results as attn_decode_ragged on the same keys."""
    batch, max_len = scratch.batch, scratch.max_len
    f32 = torch.float32
    _need(q, "q", f32, batch * Q_HEADS * DIM)
    _need(gate, "gate", f32, batch * Q_HEADS * DIM)
    _need(core, "core", f32, batch * Q_HEADS * DIM)
    _need(lens, "lens", torch.int32, batch)
    if page_table.dim() != 2 or page_table.shape[0] != batch:
        raise ValueError("page_table must be [batch][max_pages]")
    _need(page_table, "page_table", torch.int32, batch * page_table.shape[1])
    for name, t in (("k_pages", k_pages), ("v_pages", v_pages)):
        if not t.is_cuda or t.dtype not in (torch.float16, torch.int16):
            raise ValueError(f"{name} must be a float16 device tensor")
    _lib.check(_lib.load().miso_attn_decode_paged(
        _ptr(q), _ptr(gate), _ptr(k_pages), _ptr(v_pages), _ptr(page_table),
        int(page_table.shape[1]), page_size, _ptr(lens), batch, max_len, _ptr(core),
        _ptr(scratch.part_m), _ptr(scratch.part_l), _ptr(scratch.part_o), _stream(stream)))


# ------------------------------------------------------------------------------------------------
# fp8 KV cache: e4m3 rows (uint8 [2][max_ctx][256]) with one power-of-two f32 scale per row
# ([2][max_ctx]); value = scale * e4m3(code). Format contract: include/miso_attn.h.
# ------------------------------------------------------------------------------------------------

class Fp8Cache:
    """Device buffers of an e4m3 KV cache for max_ctx positions of both KV heads."""

    def __init__(self, max_ctx: int, device="cuda"):
        self.max_ctx = max_ctx
        self.k8 = torch.zeros(KV_HEADS * max_ctx * DIM, dtype=torch.uint8, device=device)
        self.v8 = torch.zeros(KV_HEADS * max_ctx * DIM, dtype=torch.uint8, device=device)
        self.k_scale = torch.zeros(KV_HEADS * max_ctx, dtype=torch.float32, device=device)
        self.v_scale = torch.zeros(KV_HEADS * max_ctx, dtype=torch.float32, device=device)

    def buffers(self):
        return self.k8, self.v8, self.k_scale, self.v_scale


def _need_fp8(cache: Fp8Cache) -> None:
    n = KV_HEADS * cache.max_ctx
    _need(cache.k8, "k8", torch.uint8, n * DIM)
    _need(cache.v8, "v8", torch.uint8, n * DIM)
    _need(cache.k_scale, "k_scale", torch.float32, n)
    _need(cache.v_scale, "v_scale", torch.float32, n)


def attn_kv_encode_fp8(k_cache, v_cache, cache: Fp8Cache, pos0: int, n: int,
                       stream=None) -> None:
    """Encode rows [pos0, pos0 + n) of both KV heads of an f16 cache into `cache`."""
    m = cache.max_ctx
    _need(k_cache, "k_cache", _cache_dtype(k_cache), KV_HEADS * m * DIM)
    _need(v_cache, "v_cache", _cache_dtype(v_cache), KV_HEADS * m * DIM)
    _need_fp8(cache)
    _lib.check(_lib.load().miso_attn_kv_encode_fp8(
        _ptr(k_cache), _ptr(v_cache), *(_ptr(b) for b in cache.buffers()), pos0, n, m,
        _stream(stream)))


def attn_prep_fp8(qg, k, v, q_norm, k_norm, inv_freq, cache: Fp8Cache, q, pos: int,
                  eps: float = 1e-6, stream=None) -> None:
    """attn_prep appending the token's K / V to `cache` as e4m3 rows at position pos."""
    f32 = torch.float32
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(k, "k", f32, KV_HEADS * DIM)
    _need(v, "v", f32, KV_HEADS * DIM)
    for name, t, n in (("q_norm", q_norm, DIM), ("k_norm", k_norm, DIM),
                       ("inv_freq", inv_freq, 32), ("q", q, Q_HEADS * DIM)):
        _need(t, name, f32, n)
    _need_fp8(cache)
    _lib.check(_lib.load().miso_attn_prep_fp8(
        _ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(inv_freq),
        *(_ptr(b) for b in cache.buffers()), _ptr(q), pos, cache.max_ctx, eps, _stream(stream)))


def attn_prep_batch_fp8(qg, k, v, q_norm, k_norm, inv_freq, cache: Fp8Cache, q, pos0: int,
                        n: int, proj_stride: int, eps: float = 1e-6, stream=None) -> None:
    """attn_prep_batch appending the tokens' K / V to `cache` as e4m3 rows at pos0 .. pos0 + n - 1;
    qg / k / v are views into a token-major projection buffer, rows proj_stride floats apart."""
    f32 = torch.float32
    for name, t in (("qg", qg), ("k", k), ("v", v)):
        if not t.is_cuda or t.dtype != f32:
            raise ValueError(f"{name} must be a float32 device tensor")
    for name, t, m in (("q_norm", q_norm, DIM), ("k_norm", k_norm, DIM),
                       ("inv_freq", inv_freq, 32), ("q", q, n * Q_HEADS * DIM)):
        _need(t, name, f32, m)
    _need_fp8(cache)
    _lib.check(_lib.load().miso_attn_prep_batch_fp8(
        _ptr(qg), _ptr(k), _ptr(v), _ptr(q_norm), _ptr(k_norm), _ptr(inv_freq),
        *(_ptr(b) for b in cache.buffers()), _ptr(q), pos0, cache.max_ctx, eps, n, proj_stride,
        _stream(stream)))


class Fp8PrefillScratch:
    """f16 workspaces for attn_prefill_fp8 over up to max_rows cache rows (pos0 + n)."""

    def __init__(self, max_rows: int, device="cuda"):
        self.max_rows = max_rows
        self.k = torch.empty(KV_HEADS * max_rows * DIM, dtype=torch.float16, device=device)
        self.v = torch.empty(KV_HEADS * max_rows * DIM, dtype=torch.float16, device=device)


def attn_prefill_fp8(q, qg, cache: Fp8Cache, core, pos0: int, n: int,
                     scratch: Optional[Fp8PrefillScratch] = None, qg_stride: int = QG_STRIDE,
                     stream=None) -> Fp8PrefillScratch:
    """attn_prefill over an e4m3 cache: rows [0, pos0 + n) widened to f16 into `scratch` (made
    here when None), then the f16 causal prefill over them. Returns the scratch used."""
    if scratch is None:
        scratch = Fp8PrefillScratch(pos0 + n, device=q.device)
    if pos0 + n > scratch.max_rows:
        raise ValueError("pos0 + n exceeds the scratch capacity")
    f32 = torch.float32
    _need(q, "q", f32, n * Q_HEADS * DIM)
    _need(qg, "qg", f32, (n - 1) * qg_stride + Q_HEADS * 2 * DIM if n else 0)
    _need(core, "core", f32, n * Q_HEADS * DIM)
    _need_fp8(cache)
    _lib.check(_lib.load().miso_attn_prefill_fp8(
        _ptr(q), _ptr(qg), *(_ptr(b) for b in cache.buffers()), _ptr(scratch.k), _ptr(scratch.v),
        _ptr(core), pos0, n, cache.max_ctx, qg_stride, _stream(stream)))
    return scratch


def attn_decode_fp8(q, qg, cache: Fp8Cache, core, scratch: DecodeScratch, length: int,
                    n_splits: Optional[int] = None, stream=None) -> int:
    """attn_decode over an e4m3 cache: split + combine over keys [0, length)."""
    if n_splits is None:
        n_splits = attn_n_splits(length, scratch.max_splits)
    if n_splits > scratch.max_splits:
        raise ValueError("n_splits exceeds the scratch capacity")
    f32 = torch.float32
    _need(q, "q", f32, Q_HEADS * DIM)
    _need(qg, "qg", f32, Q_HEADS * 2 * DIM)
    _need(core, "core", f32, Q_HEADS * DIM)
    _need_fp8(cache)
    _lib.check(_lib.load().miso_attn_decode_fp8(
        _ptr(q), _ptr(qg), *(_ptr(b) for b in cache.buffers()), _ptr(core),
        _ptr(scratch.part_m), _ptr(scratch.part_l), _ptr(scratch.part_o), length, cache.max_ctx,
        n_splits, _stream(stream)))
    return n_splits


# ------------------------------------------------------------------------------------------------
# Q4_K GEMV of the attention's projections (weights: rows of Q4_K r1 blocks, 144 bytes per 256)
# ------------------------------------------------------------------------------------------------

def q4k_gemv(w, x, y, n_rows: int, k: int, act: str = "fp16", stream=None) -> None:
    """y[:n_rows] = W x for Q4_K r1 rows w (uint8 device tensor, n_rows * k / 256 * 144 bytes)."""
    if act not in ("fp16", "int8"):
        raise ValueError("act must be 'fp16' or 'int8'")
    _need(w, "w", torch.uint8, n_rows * k // 256 * 144)
    _need(x, "x", torch.float32, k)
    _need(y, "y", torch.float32, n_rows)
    _lib.check(_lib.load().miso_attn_q4k_gemv(_ptr(w), _ptr(x), _ptr(y), n_rows, k,
                                              1 if act == "fp16" else 0, _stream(stream)))


def q6k_row_bytes(k: int) -> int:
    """Bytes of one Q6_K r1 row of k weights (210 per 256, rounded up to 16)."""
    return (k // 256 * 210 + 15) // 16 * 16


def q6k_gemv(w, x, y, n_rows: int, k: int, stream=None) -> None:
    """y[:n_rows] = W x for Q6_K r1 rows w (uint8 device tensor), f16 activations."""
    _need(w, "w", torch.uint8, n_rows * q6k_row_bytes(k))
    _need(x, "x", torch.float32, k)
    _need(y, "y", torch.float32, n_rows)
    _lib.check(_lib.load().miso_attn_q6k_gemv(_ptr(w), _ptr(x), _ptr(y), n_rows, k,
                                              _stream(stream)))


def q4k_q6k_gemv_pair(w4, n4: int, y4, w6, n6: int, y6, x, stream=None) -> None:
    """The attention's q (Q4_K, f16 activations) and v (Q6_K) projections of x (2048 floats) in
    one launch; bit-identical to q4k_gemv(..., act="fp16") and q6k_gemv on the same rows."""
    k = 2048
    _need(w4, "w4", torch.uint8, n4 * k // 256 * 144)
    _need(w6, "w6", torch.uint8, n6 * q6k_row_bytes(k))
    _need(x, "x", torch.float32, k)
    _need(y4, "y4", torch.float32, n4)
    _need(y6, "y6", torch.float32, n6)
    _lib.check(_lib.load().miso_attn_q4k_q6k_gemv_pair(_ptr(w4), n4, _ptr(y4), _ptr(w6), n6,
                                                       _ptr(y6), _ptr(x), _stream(stream)))


def qkv_gemv(wq, nq: int, yq, wk, nk: int, yk, wv, nv: int, yv, x, stream=None) -> None:
    """q and k (Q4_K, f16 activations) and v (Q6_K) projections of x (2048 floats) in one launch;
    bit-identical to the separate q4k_gemv / q6k_gemv calls."""
    k = 2048
    _need(wq, "wq", torch.uint8, nq * k // 256 * 144)
    _need(wk, "wk", torch.uint8, nk * k // 256 * 144)
    _need(wv, "wv", torch.uint8, nv * q6k_row_bytes(k))
    _need(x, "x", torch.float32, k)
    for name, t, n in (("yq", yq, nq), ("yk", yk, nk), ("yv", yv, nv)):
        _need(t, name, torch.float32, n)
    _lib.check(_lib.load().miso_attn_qkv_gemv(_ptr(wq), nq, _ptr(yq), _ptr(wk), nk, _ptr(yk),
                                              _ptr(wv), nv, _ptr(yv), _ptr(x), _stream(stream)))


# ------------------------------------------------------------------------------------------------
# Prefill projection GEMMs (src/engine/weights.hpp:78-90: GemmInput, gemm_input, gemm)
# ------------------------------------------------------------------------------------------------

class GemmInput:
    """Activations of a token chunk prepared for the prefill GEMMs (the reference's GemmInput,
    src/engine/weights.hpp:78-84): xh, max_tok x max_k f16 values, and xs, their per-32 sums."""

    def __init__(self, max_tok: int, max_k: int, device="cuda"):
        self.xh = torch.empty(max_tok * max_k, dtype=torch.float16, device=device)
        self.xs = torch.empty(max_tok * max_k // 32, dtype=torch.float32, device=device)
        self.k = 0
        self.n_tok = 0


def gemm_input(x, k: int, n_tok: int, inp: GemmInput, stream=None) -> None:
    """Prepares x ([n_tok][k] floats) as GEMM input (src/engine/weights.hip:306-314)."""
    if n_tok * k > inp.xh.numel() or k % 256 != 0:
        raise RuntimeError("gemm_input: chunk does not fit")
    _need(x, "x", torch.float32, n_tok * k)
    inp.k, inp.n_tok = k, n_tok
    _lib.check(_lib.load().miso_attn_gemm_input(_ptr(x), _ptr(inp.xh), _ptr(inp.xs), k, n_tok,
                                                _stream(stream)))


GEMM_FORMATS = {"q4_k": 0, "q6_k": 1}


def gemm(w, fmt: str, n_rows: int, k: int, inp: GemmInput, y, ldy: int, stream=None) -> None:
    """Y[t][n] = W x[t] for the prepared chunk, row t of Y at y + t * ldy (src/engine/weights.hip:
    316-330). w: n_rows rows of k weights in the Q4_K r1 ("q4_k") or Q6_K r1 ("q6_k") layout."""
    if k != inp.k:
        raise RuntimeError("gemm: K mismatch")
    if fmt not in GEMM_FORMATS:
        raise RuntimeError("gemm: unsupported type")
    row = k // 256 * 144 if fmt == "q4_k" else q6k_row_bytes(k)
    _need(w, "w", torch.uint8, n_rows * row)
    if inp.n_tok:
        _need(y, "y", torch.float32, (inp.n_tok - 1) * ldy + n_rows)
    _lib.check(_lib.load().miso_attn_gemm(_ptr(w), GEMM_FORMATS[fmt], _ptr(inp.xh), _ptr(inp.xs),
                                          _ptr(y), k, n_rows, inp.n_tok, ldy, _stream(stream)))


# ------------------------------------------------------------------------------------------------
# One attention layer step (src/engine/attention.hip:76-148), engine sizing retuned for MI355X
# ------------------------------------------------------------------------------------------------

LAYER_MAX_SPLITS = 128        # decode split cap (reference: 60, src/engine/attention.hpp:46)
LAYER_MAX_CHUNK = 4096        # prefill chunk (reference: 512, src/engine/model.hpp:58)
LAYER_PREFILL_MIN_TOKENS = 12  # prefill from this many tokens (reference: 8, model.hpp:80)


class _QMatrix(ctypes.Structure):
    _fields_ = [("w", ctypes.c_void_p), ("format", ctypes.c_int32), ("n_rows", ctypes.c_uint32),
                ("k", ctypes.c_uint32)]


class _Layer(ctypes.Structure):
    _fields_ = [("q", _QMatrix), ("k", _QMatrix), ("v", _QMatrix), ("o", _QMatrix),
                ("attn_norm", ctypes.c_void_p), ("q_norm", ctypes.c_void_p),
                ("k_norm", ctypes.c_void_p), ("inv_freq", ctypes.c_void_p)]


class Layer:
    """One attention layer's device weights: (r1 bytes, "q4_k" | "q6_k") for q (8192 x 2048), k and
    v (512 x 2048) and o (2048 x 4096); attn_norm [2048], q_norm / k_norm [256], inv_freq [32]
    (float32). Keeps the tensors alive for the C description it holds."""

    SHAPES = {"q": (8192, 2048), "k": (512, 2048), "v": (512, 2048), "o": (2048, 4096)}

    def __init__(self, q, k, v, o, attn_norm, q_norm, k_norm, inv_freq):
        self._keep = (q, k, v, o, attn_norm, q_norm, k_norm, inv_freq)
        mats = {}
        for name, (t, fmt) in (("q", q), ("k", k), ("v", v), ("o", o)):
            if fmt not in GEMM_FORMATS:
                raise ValueError(f"{name}: format must be 'q4_k' or 'q6_k'")
            n, kk = self.SHAPES[name]
            row = kk // 256 * 144 if fmt == "q4_k" else q6k_row_bytes(kk)
            _need(t, name, torch.uint8, n * row)
            mats[name] = _QMatrix(_ptr(t), GEMM_FORMATS[fmt], n, kk)
        for name, t, n in (("attn_norm", attn_norm, 2048), ("q_norm", q_norm, DIM),
                           ("k_norm", k_norm, DIM), ("inv_freq", inv_freq, 32)):
            _need(t, name, torch.float32, n)
        self.c = _Layer(mats["q"], mats["k"], mats["v"], mats["o"], _ptr(attn_norm),
                        _ptr(q_norm), _ptr(k_norm), _ptr(inv_freq))


class LayerWorkspace:
    """Device workspaces of the layer steps: decode, and prefill chunks of up to max_tok tokens."""

    def __init__(self, max_tok: int = LAYER_MAX_CHUNK, device="cuda"):
        lib = _lib.load()
        self.max_tok = max_tok
        self.decode = torch.empty(int(lib.miso_attn_layer_decode_ws()), dtype=torch.float32,
                                  device=device)
        # zero-filled once: the balanced prefill's pair counters sit at its end
        self.prefill = torch.zeros(max(1, int(lib.miso_attn_layer_prefill_ws(max_tok))),
                                   dtype=torch.float32, device=device)
        # the attention output before the output projection (the engine's scratch.core /
        # ps.core): the last decode step's [16 * 256], the last prefill chunk's [n][16 * 256]
        at = int(lib.miso_attn_layer_decode_core())
        self.decode_core = self.decode[at:at + 4096]
        at = int(lib.miso_attn_layer_prefill_core(max_tok))
        self.prefill_core = self.prefill[at:at + max_tok * 4096].view(max_tok, 4096)


def _layer_cache(k_cache, v_cache, max_ctx: int):
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _need(t, name, _cache_dtype(t), KV_HEADS * max_ctx * DIM)
    return _ptr(k_cache), _ptr(v_cache)


def layer_decode(layer: Layer, k_cache, v_cache, max_ctx: int, length: int, h, delta, y,
                 eps: float, ws: LayerWorkspace, stream=None) -> None:
    """The token at position `length`: h += delta (delta may be None), y = the layer's output;
    K/V appended at `length` (src/engine/attention.hip:76-114)."""
    _need(h, "h", torch.float32, 2048)
    _need(y, "y", torch.float32, 2048)
    if delta is not None:
        _need(delta, "delta", torch.float32, 2048)
    kc, vc = _layer_cache(k_cache, v_cache, max_ctx)
    _lib.check(_lib.load().miso_attn_layer_decode(
        ctypes.addressof(layer.c), kc, vc, length, max_ctx, _ptr(h), _ptr(delta), _ptr(y), eps,
        _ptr(ws.decode), _stream(stream)))


def _rows(n: int, **tensors):
    for name, t in tensors.items():
        if t is not None:
            _need(t, name, torch.float32, n * 2048)


def layer_prefill(layer: Layer, k_cache, v_cache, max_ctx: int, pos0: int, n: int, h, delta, y,
                  eps: float, ws: LayerWorkspace, stream=None) -> None:
    """n tokens at pos0 ([n][2048] h / delta / y) in one prefill step
    (src/engine/attention.hip:116-148)."""
    _rows(n, h=h, delta=delta, y=y)
    kc, vc = _layer_cache(k_cache, v_cache, max_ctx)
    _lib.check(_lib.load().miso_attn_layer_prefill(
        ctypes.addressof(layer.c), kc, vc, pos0, n, max_ctx, _ptr(h), _ptr(delta), _ptr(y), eps,
        _ptr(ws.prefill), ws.max_tok, _stream(stream)))


def layer_ingest(layer: Layer, k_cache, v_cache, max_ctx: int, pos0: int, n: int, h, delta, y,
                 eps: float, ws: LayerWorkspace, chunk: int = 0, stream=None) -> None:
    """n tokens at pos0 with the engine's policy: one decode step per token below
    LAYER_PREFILL_MIN_TOKENS, otherwise prefill chunks of min(chunk or LAYER_MAX_CHUNK,
    ws.max_tok) tokens."""
    _rows(n, h=h, delta=delta, y=y)
    kc, vc = _layer_cache(k_cache, v_cache, max_ctx)
    _lib.check(_lib.load().miso_attn_layer_ingest(
        ctypes.addressof(layer.c), kc, vc, pos0, n, max_ctx, _ptr(h), _ptr(delta), _ptr(y), eps,
        _ptr(ws.decode), _ptr(ws.prefill), ws.max_tok, chunk, _stream(stream)))
