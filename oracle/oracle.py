"""Python wrapper of the CPU oracle (oracle/attn_oracle.c) and of the reference kernels built
from the reference's own sources (oracle/_ref).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product (miso_amd/) never imports this module.

Each function cites the reference code it restates in attn_oracle.c's header.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libattn_oracle.so"
REF_PATH = HERE / "_ref" / "libmiso_ref_kernels.so"

Q_HEADS, KV_HEADS, DIM, GROUP = 16, 2, 256, 8
QG_STRIDE = Q_HEADS * 2 * DIM

_lib = None


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(c_void_p)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: run `make -C oracle`")
        L = ctypes.CDLL(str(LIB_PATH))
        V = c_void_p
        sig = {
            "oracle_splitmix64": (c_uint64, [POINTER(c_uint64)]),
            "oracle_xoshiro_stream": (None, [c_uint64, V, ctypes.c_size_t]),
            "oracle_xoshiro_raw": (None, [V, V, ctypes.c_size_t]),
            "oracle_fill_normal": (None, [c_uint64, c_float, V, ctypes.c_size_t]),
            "oracle_fill_normal_f16": (None, [c_uint64, V, ctypes.c_size_t]),
            "oracle_f32_to_f16": (c_uint16, [c_float]),
            "oracle_f16_to_f32": (c_float, [c_uint16]),
            "oracle_f32_to_f16_array": (None, [V, V, ctypes.c_size_t]),
            "oracle_f16_to_f32_array": (None, [V, V, ctypes.c_size_t]),
            "oracle_decode_f64": (None, [V, V, V, V, c_uint32, c_uint32, V, c_int]),
            "oracle_ragged_f64": (None, [V, V, V, V, V, V, c_uint32, V, c_int]),
            "oracle_prefill_f64": (None, [V, V, c_uint32, V, V, c_uint32, c_uint32, V, c_uint32,
                                          V, c_int]),
            "oracle_partials_f64": (None, [V, V, V, c_uint32, c_uint32, c_uint32, c_uint32, V, V,
                                           V]),
            "oracle_combine_f32": (None, [V, V, V, V, c_uint32, V]),
            "oracle_inv_freq": (None, [c_float, V]),
            "oracle_prep_f64": (None, [V, V, V, V, V, V, c_uint32, c_float, V, V, V]),
            "oracle_ref_n_splits": (c_uint32, [c_uint32, c_uint32]),
            "oracle_e4m3_value": (c_double, [ctypes.c_uint8]),
            "oracle_e4m3_encode": (ctypes.c_uint8, [c_float]),
            "oracle_fp8_encode_rows": (None, [V, ctypes.c_size_t, V, V]),
            "oracle_decode_fp8_f64": (None, [V, V, V, V, V, V, c_uint32, c_uint32, V, c_int]),
            "oracle_q4k_dequant": (None, [V, ctypes.c_size_t, V, V]),
            "oracle_q4k_mins": (None, [V, ctypes.c_size_t, V]),
            "oracle_q4k_repack_r1": (None, [V, ctypes.c_size_t, V]),
            "oracle_q4k_gemv_f64": (None, [V, V, c_uint32, c_uint32, V]),
            "oracle_q6k_dequant": (None, [V, ctypes.c_size_t, V]),
            "oracle_q6k_repack_r1": (None, [V, c_uint32, c_uint32, V]),
            "oracle_q6k_gemv_f64": (None, [V, V, c_uint32, c_uint32, V]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


# ------------------------------------------------------------------------------------------------
# Generator and binary16
# ------------------------------------------------------------------------------------------------

def splitmix64_stream(seed: int, n: int) -> np.ndarray:
    st = c_uint64(seed)
    return np.array([lib().oracle_splitmix64(ctypes.byref(st)) for _ in range(n)], dtype=np.uint64)


def xoshiro_stream(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint64)
    lib().oracle_xoshiro_stream(seed, _ptr(out), n)
    return out


def xoshiro_raw(state, n: int) -> np.ndarray:
    st = np.ascontiguousarray(state, dtype=np.uint64)
    out = np.empty(n, dtype=np.uint64)
    lib().oracle_xoshiro_raw(_ptr(st), _ptr(out), n)
    return out


def normal(seed: int, n: int, scale: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().oracle_fill_normal(seed, scale, _ptr(out), n)
    return out


def normal_f16(seed: int, n: int) -> np.ndarray:
    """binary16 bit patterns (uint16) of N(0,1) values."""
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_fill_normal_f16(seed, _ptr(out), n)
    return out


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_f16_array(_ptr(a), _ptr(out), a.size)
    return out


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().oracle_f16_to_f32_array(_ptr(h), _ptr(out), h.size)
    return out


# ------------------------------------------------------------------------------------------------
# Seeded inputs of the configs (identical on every machine)
# ------------------------------------------------------------------------------------------------

def decode_inputs(seed: int, length: int, max_ctx: int | None = None, q_scale: float = 1.0):
    """q [16][256] = q_scale * N(0,1); qg [16][512] N(0,1) (gate = second half of each head);
    K/V caches [2][max_ctx][256] binary16 of N(0,1). Streams: seed*8 + {0,1,2,3}."""
    max_ctx = length if max_ctx is None else max_ctx
    return {
        "q": normal(seed * 8 + 0, Q_HEADS * DIM, q_scale),
        "qg": normal(seed * 8 + 1, Q_HEADS * 2 * DIM),
        "k": normal_f16(seed * 8 + 2, KV_HEADS * max_ctx * DIM),
        "v": normal_f16(seed * 8 + 3, KV_HEADS * max_ctx * DIM),
        "len": length,
        "max_ctx": max_ctx,
    }


def prefill_inputs(seed: int, pos0: int, n: int, max_ctx: int | None = None,
                   q_scale: float = 1.0, qg_stride: int = QG_STRIDE):
    """q [n][16][256]; qg [n][qg_stride] N(0,1) (gate of head h at h*512 + 256); K/V caches
    [2][max_ctx][256] holding keys [0, pos0 + n) (whole cache filled)."""
    max_ctx = pos0 + n if max_ctx is None else max_ctx
    return {
        "q": normal(seed * 8 + 4, n * Q_HEADS * DIM, q_scale),
        "qg": normal(seed * 8 + 5, n * qg_stride),
        "k": normal_f16(seed * 8 + 6, KV_HEADS * max_ctx * DIM),
        "v": normal_f16(seed * 8 + 7, KV_HEADS * max_ctx * DIM),
        "pos0": pos0,
        "n": n,
        "max_ctx": max_ctx,
        "qg_stride": qg_stride,
    }


def ragged_lengths(seed: int, batch: int, lo: int, hi: int) -> np.ndarray:
    """Lengths uniform in [lo, hi] from the xoshiro stream of `seed`."""
    raw = xoshiro_stream(seed, batch)
    return (lo + (raw % np.uint64(hi - lo + 1))).astype(np.uint32)


def ragged_inputs(seed: int, lens: np.ndarray):
    lens = np.asarray(lens, dtype=np.uint32)
    batch = lens.size
    sizes = lens.astype(np.uint64) * np.uint64(KV_HEADS * DIM)
    offsets = np.zeros(batch, dtype=np.uint64)
    offsets[1:] = np.cumsum(sizes)[:-1]
    total = int(sizes.sum())
    return {
        "q": normal(seed * 8 + 0, batch * Q_HEADS * DIM),
        "gate": normal(seed * 8 + 1, batch * Q_HEADS * DIM),
        "k": normal_f16(seed * 8 + 2, total),
        "v": normal_f16(seed * 8 + 3, total),
        "lens": lens,
        "offsets": offsets,
    }


# ------------------------------------------------------------------------------------------------
# References
# ------------------------------------------------------------------------------------------------

def decode_f64(q, qg, k, v, length: int, max_ctx: int, threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    qg = np.ascontiguousarray(qg, np.float32)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    out = np.empty((Q_HEADS, DIM), dtype=np.float64)
    lib().oracle_decode_f64(_ptr(q), _ptr(qg), _ptr(k), _ptr(v), length, max_ctx, _ptr(out),
                            threads or default_threads())
    return out


# ------------------------------------------------------------------------------------------------
# e4m3 KV rows (the format of miso_amd/kernels/attention_decode_fp8.hpp; no reference counterpart)
# ------------------------------------------------------------------------------------------------

def e4m3_table() -> np.ndarray:
    """Value of each of the 256 e4m3 codes (NaN for 0x7F / 0xFF)."""
    return np.array([lib().oracle_e4m3_value(c) for c in range(256)], dtype=np.float64)


def e4m3_encode(y: float) -> int:
    """Nearest e4m3 code of y (|y| < 256), ties to even, found by search."""
    return int(lib().oracle_e4m3_encode(float(y)))


def fp8_encode_rows(x) -> tuple[np.ndarray, np.ndarray]:
    """Rows of 256 floats -> (codes uint8 [rows, 256], power-of-two scales float32 [rows])."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1, DIM)
    codes = np.empty(x.shape, dtype=np.uint8)
    scales = np.empty(x.shape[0], dtype=np.float32)
    lib().oracle_fp8_encode_rows(_ptr(x), x.shape[0], _ptr(codes), _ptr(scales))
    return codes, scales


def fp8_dequant(codes, scales) -> np.ndarray:
    """value = scale * e4m3(code), in float64, shape of codes."""
    codes = np.asarray(codes, np.uint8)
    return e4m3_table()[codes] * np.asarray(scales, np.float64).reshape(
        codes.shape[:-1] + (1,))


def decode_fp8_f64(q, qg, k8, v8, ks, vs, length: int, max_ctx: int,
                   threads: int = 0) -> np.ndarray:
    """decode_f64 over e4m3 rows: k8 / v8 [2][max_ctx][256] uint8, ks / vs [2][max_ctx]."""
    q = np.ascontiguousarray(q, np.float32)
    qg = np.ascontiguousarray(qg, np.float32)
    k8 = np.ascontiguousarray(k8, np.uint8)
    v8 = np.ascontiguousarray(v8, np.uint8)
    ks = np.ascontiguousarray(ks, np.float32)
    vs = np.ascontiguousarray(vs, np.float32)
    rows = KV_HEADS * max_ctx
    if min(k8.size, v8.size) < rows * DIM or min(ks.size, vs.size) < rows or length > max_ctx:
        raise ValueError("e4m3 rows / scales smaller than [2][max_ctx] (or length > max_ctx)")
    out = np.empty((Q_HEADS, DIM), dtype=np.float64)
    lib().oracle_decode_fp8_f64(_ptr(q), _ptr(qg), _ptr(k8), _ptr(v8), _ptr(ks), _ptr(vs),
                                length, max_ctx, _ptr(out), threads or default_threads())
    return out


# ------------------------------------------------------------------------------------------------
# Q4_K projection weights (GGUF blocks of 144 bytes per 256 weights)
# ------------------------------------------------------------------------------------------------

def q4k_dequant(blocks) -> tuple[np.ndarray, np.ndarray]:
    """GGUF Q4_K blocks -> (f32 weights, d * sc of each weight's sub-block)."""
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    nb = blocks.size // 144
    w = np.empty(nb * 256, np.float32)
    ds = np.empty(nb * 256, np.float32)
    lib().oracle_q4k_dequant(_ptr(blocks), nb, _ptr(w), _ptr(ds))
    return w, ds


def q4k_mins(blocks) -> np.ndarray:
    """GGUF Q4_K blocks -> dmin * m of each weight's sub-block (f32)."""
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    nb = blocks.size // 144
    dm = np.empty(nb * 256, np.float32)
    lib().oracle_q4k_mins(_ptr(blocks), nb, _ptr(dm))
    return dm


def qgemm_act_ref(x) -> tuple[np.ndarray, np.ndarray]:
    """The prefill GEMM's activation prep, the reference's CPU rule (tests/test_qgemm.hip:92-104):
    h = x rounded to f16 (RNE); per 32-group the f32 sum, added in order to 0, of the chunk sums
    ((h0 + h1) + h2) + h3 of its 8 four-element chunks. Returns (h as float16, sums as float32)."""
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    h = x.astype(np.float16)
    g = h.astype(np.float32).reshape(-1, 32)
    s = np.zeros(g.shape[0], np.float32)
    for c in range(8):
        q = g[:, 4 * c:4 * c + 4]
        s = s + (((q[:, 0] + q[:, 1]) + q[:, 2]) + q[:, 3])
    return h, s


def q4k_repack_r1(blocks) -> np.ndarray:
    """GGUF Q4_K blocks -> the r1 layout the GPU GEMV reads."""
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    out = np.empty_like(blocks)
    lib().oracle_q4k_repack_r1(_ptr(blocks), blocks.size // 144, _ptr(out))
    return out


def q4k_gemv_f64(blocks, x, n_rows: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n_rows, np.float64)
    lib().oracle_q4k_gemv_f64(_ptr(blocks), _ptr(x), n_rows, k, _ptr(y))
    return y


def q6k_dequant(blocks) -> np.ndarray:
    """GGUF Q6_K blocks (210 bytes per 256 weights) -> f32 weights."""
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    w = np.empty(blocks.size // 210 * 256, np.float32)
    lib().oracle_q6k_dequant(_ptr(blocks), blocks.size // 210, _ptr(w))
    return w


def q6k_repack_r1(blocks, n_rows: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    out = np.empty(n_rows * ((k // 256 * 210 + 15) // 16 * 16), np.uint8)
    lib().oracle_q6k_repack_r1(_ptr(blocks), n_rows, k, _ptr(out))
    return out


def q6k_gemv_f64(blocks, x, n_rows: int, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(n_rows, np.float64)
    lib().oracle_q6k_gemv_f64(_ptr(blocks), _ptr(x), n_rows, k, _ptr(y))
    return y


def q4k_error_bound(w, ds, x, act: str) -> np.ndarray:
    """Per-row bound on |y_gpu - W x| for f32 dequantized rows w [n][k], the same rule as
    tests/test_q4k_gemv.hip:60-90: activation conversion error (fp16: 2^-11 |x| + 2^-25; int8:
    half a step of the per-32 absmax / 127 grid) times |W|, the fp16 nibble chain term
    2^-20 * 15 * d sc |x|, and K * 2^-23 * sum |W x| of f32 accumulation."""
    w = np.asarray(w, np.float64)
    x64 = np.asarray(x, np.float64)
    k = x64.size
    if act == "fp16":
        e = np.abs(x64) * 2.0 ** -11 + 2.0 ** -25
    else:
        amax = np.abs(x64).reshape(-1, 32).max(axis=1)
        e = np.repeat(0.5 * amax / 127.0, 32)
    bound = np.abs(w) @ e + k * 2.0 ** -23 * (np.abs(w) @ np.abs(x64))
    if act == "fp16":
        bound += 2.0 ** -20 * 15.0 * (np.asarray(ds, np.float64).reshape(w.shape) @ np.abs(x64))
    return bound


def prefill_f64(q, qg, qg_stride: int, k, v, pos0: int, max_ctx: int, tokens,
                threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    qg = np.ascontiguousarray(qg, np.float32)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    tok = np.ascontiguousarray(tokens, dtype=np.uint32)
    out = np.empty((tok.size, Q_HEADS, DIM), dtype=np.float64)
    lib().oracle_prefill_f64(_ptr(q), _ptr(qg), qg_stride, _ptr(k), _ptr(v), pos0, max_ctx,
                             _ptr(tok), tok.size, _ptr(out), threads or default_threads())
    return out


def ragged_f64(q, gate, k, v, offsets, lens, threads: int = 0) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    gate = np.ascontiguousarray(gate, np.float32)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    offsets = np.ascontiguousarray(offsets, np.uint64)
    lens = np.ascontiguousarray(lens, np.uint32)
    out = np.empty((lens.size, Q_HEADS, DIM), dtype=np.float64)
    lib().oracle_ragged_f64(_ptr(q), _ptr(gate), _ptr(k), _ptr(v), _ptr(offsets), _ptr(lens),
                            lens.size, _ptr(out), threads or default_threads())
    return out


def partials_f64(q, k, v, kvh: int, max_ctx: int, j0: int, j1: int):
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.uint16)
    v = np.ascontiguousarray(v, np.uint16)
    m = np.empty(GROUP, np.float64)
    l = np.empty(GROUP, np.float64)
    o = np.empty((GROUP, DIM), np.float64)
    lib().oracle_partials_f64(_ptr(q), _ptr(k), _ptr(v), kvh, max_ctx, j0, j1, _ptr(m), _ptr(l),
                              _ptr(o))
    return m, l, o


def combine_f32(pm, pl, po, qg, n_splits: int) -> np.ndarray:
    pm = np.ascontiguousarray(pm, np.float32)
    pl = np.ascontiguousarray(pl, np.float32)
    po = np.ascontiguousarray(po, np.float32)
    qg = np.ascontiguousarray(qg, np.float32)
    out = np.empty((Q_HEADS, DIM), np.float32)
    lib().oracle_combine_f32(_ptr(pm), _ptr(pl), _ptr(po), _ptr(qg), n_splits, _ptr(out))
    return out


def inv_freq(base: float) -> np.ndarray:
    out = np.empty(32, np.float32)
    lib().oracle_inv_freq(base, _ptr(out))
    return out


def prep_f64(qg, k, v, q_norm, k_norm, inv_freq_arr, pos: int, eps: float):
    """One token: returns (q [16][256] float64, k_f16 [2][256] uint16, v_f16 [2][256] uint16)."""
    arrs = [np.ascontiguousarray(a, np.float32) for a in (qg, k, v, q_norm, k_norm, inv_freq_arr)]
    q_out = np.empty((Q_HEADS, DIM), np.float64)
    k_out = np.empty((KV_HEADS, DIM), np.uint16)
    v_out = np.empty((KV_HEADS, DIM), np.uint16)
    lib().oracle_prep_f64(*[_ptr(a) for a in arrs], pos, eps, _ptr(q_out), _ptr(k_out),
                          _ptr(v_out))
    return q_out, k_out, v_out


def rmsnorm_f64(h, weight, eps: float) -> np.ndarray:
    """The reference's residual RMSNorm (kernels/rmsnorm.hpp:2-4,40-47) in float64, per row:
    h / sqrt(mean(h^2) + eps) * weight (the GGUF weight already stores 1 + w)."""
    h = np.asarray(h, np.float64)
    r = 1.0 / np.sqrt((h * h).mean(axis=-1, keepdims=True) + float(eps))
    return h * r * np.asarray(weight, np.float64)


def layer_f64(h, delta, wq, wk, wv, wo, attn_norm, q_norm, k_norm, inv_freq_arr, pos0: int,
              max_ctx: int, eps: float, k16=None, v16=None, with_core: bool = False):
    """One gated attention layer over T consecutive tokens at pos0..pos0 + T - 1 (the engine's
    attention_decode / attention_prefill, src/engine/attention.hip:76-148, token by token):
    h += delta; xn = RMSNorm(h) attn_norm; [q + gate | k | v] = W xn with xn rounded to f16 (the
    reference's GEMV and GEMM take f16 activations: kernels/q4k_gemv.hpp ActFormat::Fp16,
    kernels/qgemm.hpp qgemm_act); per-head norms, RoPE and the f16 K/V append (prep_f64);
    attention over the cache up to the token (decode_f64); y = W_o core with core rounded to f16.
    w*: dequantized float matrices [rows][k]. k16 / v16: the f16 caches [2][max_ctx][256]
    (updated; new zero caches when None). Returns (h, y [T][2048] float64, k16, v16), and with
    with_core also core [T][4096] float64 (the gated attention output before W_o: the engine's
    scratch.core, src/engine/attention.hpp:48)."""
    h = np.asarray(h, np.float32).reshape(-1, 2048).copy()
    if delta is not None:
        h = (h + np.asarray(delta, np.float32).reshape(-1, 2048)).astype(np.float32)
    n_tok = h.shape[0]
    if k16 is None:
        k16 = np.zeros((KV_HEADS, max_ctx, DIM), np.uint16)
        v16 = np.zeros((KV_HEADS, max_ctx, DIM), np.uint16)
    xn = rmsnorm_f64(h, attn_norm, eps).astype(np.float32).astype(np.float16).astype(np.float64)
    proj = np.concatenate([xn @ np.asarray(w, np.float64).T for w in (wq, wk, wv)], axis=1)
    proj = proj.astype(np.float32)
    core = np.empty((n_tok, Q_HEADS * DIM), np.float64)
    for t in range(n_tok):
        pos = pos0 + t
        qg, kk, vv = proj[t, :8192], proj[t, 8192:8704], proj[t, 8704:]
        q, k_new, v_new = prep_f64(qg, kk, vv, q_norm, k_norm, inv_freq_arr, pos, eps)
        k16[:, pos] = k_new
        v16[:, pos] = v_new
        core[t] = decode_f64(q.astype(np.float32), qg, k16.reshape(-1), v16.reshape(-1), pos + 1,
                             max_ctx).reshape(-1)
    core16 = core.astype(np.float32).astype(np.float16).astype(np.float64)
    y = core16 @ np.asarray(wo, np.float64).T
    if with_core:
        return h, y, k16, v16, core
    return h, y, k16, v16


def ref_n_splits(length: int, max_splits: int) -> int:
    return int(lib().oracle_ref_n_splits(length, max_splits))


# ------------------------------------------------------------------------------------------------
# Tolerance of the north star: |got - ref| <= 2e-3 + 1e-2 |ref| per element (f32 output)
# ------------------------------------------------------------------------------------------------

ATOL, RTOL = 2e-3, 1e-2


def compare(got: np.ndarray, ref: np.ndarray, atol: float = ATOL, rtol: float = RTOL) -> dict:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    big = np.abs(ref) >= atol / rtol
    rel = err[big] / np.abs(ref[big]) if big.any() else np.zeros(1)
    bad = err > atol + rtol * np.abs(ref)
    finite = bool(np.isfinite(got).all())
    return {
        "ok": finite and not bool(bad.any()),
        "finite": finite,
        "max_abs": float(err.max()) if err.size else 0.0,
        "max_rel": float(rel.max()) if rel.size else 0.0,
        "n_bad": int(bad.sum()),
        "rel_l2": float(np.sqrt(((got - ref) ** 2).sum() / max((ref ** 2).sum(), 1e-300))),
        "rel_l2_head": rel_l2_rows(got, ref),
    }


def rel_l2_rows(got: np.ndarray, ref: np.ndarray) -> float:
    """Worst relative L2 error over the 256-float rows (one (token, head) output each): the
    reference's own decode and prefill gate (tests/test_attn_splitk.hip:168-174, :259-267),
    <= 1e-5 there. Rows whose reference is all zero are skipped."""
    got = np.asarray(got, np.float64).reshape(-1, 256)
    ref = np.asarray(ref, np.float64).reshape(-1, 256)
    num = ((got - ref) ** 2).sum(axis=1)
    den = (ref ** 2).sum(axis=1)
    ok = den > 0
    return float(np.sqrt(num[ok] / den[ok]).max()) if ok.any() else 0.0


# ------------------------------------------------------------------------------------------------
# The reference's kernels compiled from its sources (GPU; optional second checker)
# ------------------------------------------------------------------------------------------------

_ref = None


def ref_kernels():
    """ctypes handle of oracle/_ref/libmiso_ref_kernels.so, or None if it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        L = ctypes.CDLL(str(REF_PATH))
        V, U = c_void_p, c_uint32
        sig = {
            "ref_attn_n_splits": (U, [U, U]),
            "ref_attn_split": (c_int, [V, V, V, V, V, V, U, U, U]),
            "ref_attn_combine": (c_int, [c_int, V, V, V, V, V, U]),
            "ref_attn_prefill": (c_int, [V, V, V, V, V, U, U, U, U]),
            "ref_attn_prep": (c_int, [V, V, V, V, V, V, V, V, V, U, U, c_float]),
            "ref_attn_prep_batch": (c_int, [V, V, V, V, V, V, V, V, V, U, U, c_float, U, U]),
            "ref_qgemm_act": (c_int, [V, V, V, U, U]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _ref = L
    return _ref
