"""ctypes binding of libmiso_attn.so (the C ABI declared in include/miso_attn.h).

Loading never falls back to anything: if the built library is missing, importing the operator
module raises, naming the build command.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_uint32, c_uint64, c_void_p, c_char_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmiso_attn.so"

# name -> (restype, argtypes); must match include/miso_attn.h exactly.
P = c_void_p
SIGNATURES = {
    "miso_attn_last_error": (c_char_p, []),
    "miso_attn_version": (c_char_p, []),
    "miso_attn_n_splits": (c_uint32, [c_uint32, c_uint32]),
    "miso_attn_prefill_items": (c_uint32, [c_uint32]),
    "miso_attn_prep": (c_int, [P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_float, P]),
    "miso_attn_prep_batch": (c_int, [P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_float,
                                     c_uint32, c_uint32, P]),
    "miso_attn_split": (c_int, [P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_split_valu": (c_int, [P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_combine": (c_int, [P, P, P, P, P, c_uint32, P]),
    "miso_attn_combine_variant": (c_int, [c_int, P, P, P, P, P, c_uint32, c_uint32, c_uint32,
                                          c_uint32, P]),
    "miso_attn_decode": (c_int, [P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_decode_fused": (c_int, [P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_decode_f16q": (c_int, [P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_decode_noalloc": (c_int, [P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_prefill": (c_int, [P, P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_prefill_workspace_bytes": (c_uint64, [c_uint32]),
    "miso_attn_prefill_ws": (c_int, [P, P, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, P,
                                     c_uint64, P]),
    "miso_attn_ragged_splits": (c_uint32, [c_uint32]),
    "miso_attn_ragged_partials": (c_uint64, [c_uint32, c_uint32]),
    "miso_attn_ragged_chunk": (c_uint32, [c_uint32, c_uint32]),
    "miso_attn_decode_ragged": (c_int, [P, P, P, P, P, P, c_uint32, c_uint32, P, P, P, P, P]),
    "miso_attn_decode_paged": (c_int, [P, P, P, P, P, c_uint32, c_uint32, P, c_uint32, c_uint32,
                                       P, P, P, P, P]),
    "miso_attn_kv_encode_fp8": (c_int, [P, P, P, P, P, P, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_prep_fp8": (c_int, [P, P, P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_float,
                                   P]),
    "miso_attn_decode_fp8": (c_int, [P, P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32,
                                     P]),
    "miso_attn_prep_batch_fp8": (c_int, [P, P, P, P, P, P, P, P, P, P, P, c_uint32, c_uint32,
                                         c_float, c_uint32, c_uint32, P]),
    "miso_attn_prefill_fp8": (c_int, [P, P, P, P, P, P, P, P, P, c_uint32, c_uint32, c_uint32,
                                      c_uint32, P]),
    "miso_attn_q4k_gemv": (c_int, [P, P, P, c_uint32, c_uint32, c_int, P]),
    "miso_attn_q6k_gemv": (c_int, [P, P, P, c_uint32, c_uint32, P]),
    "miso_attn_q4k_q6k_gemv_pair": (c_int, [P, c_uint32, P, P, c_uint32, P, P, P]),
    "miso_attn_qkv_gemv": (c_int, [P, c_uint32, P, P, c_uint32, P, P, c_uint32, P, P, P]),
    "miso_attn_gemm_input": (c_int, [P, P, P, c_uint32, c_uint32, P]),
    "miso_attn_gemm": (c_int, [P, c_int, P, P, P, c_uint32, c_uint32, c_uint32, c_uint32, P]),
    "miso_attn_layer_decode_ws": (c_uint64, []),
    "miso_attn_layer_prefill_ws": (c_uint64, [c_uint32]),
    "miso_attn_layer_decode_core": (c_uint64, []),
    "miso_attn_layer_prefill_core": (c_uint64, [c_uint32]),
    "miso_attn_layer_decode": (c_int, [P, P, P, c_uint32, c_uint32, P, P, P, c_float, P, P]),
    "miso_attn_layer_prefill": (c_int, [P, P, P, c_uint32, c_uint32, c_uint32, P, P, P, c_float,
                                        P, c_uint32, P]),
    "miso_attn_layer_ingest": (c_int, [P, P, P, c_uint32, c_uint32, c_uint32, P, P, P, c_float,
                                       P, P, c_uint32, c_uint32, P]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load (once) and type the library. Raises RuntimeError if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m miso_amd.build` "
            "(or __graft_entry__.build()); there is no fallback path")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message for a non-zero return code (the reference
    throws std::runtime_error for the same failures)."""
    if rc != 0:
        msg = load().miso_attn_last_error().decode()
        raise RuntimeError(msg or f"miso_attn call failed with code {rc}")
