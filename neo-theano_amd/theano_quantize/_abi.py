"""ctypes binding of libtq.so's C ABI (include/tq.h).

This is the Python-side counterpart of the theano-rocm FFI block: it loads the
in-tree libtq.so, declares every entry point's signature and turns status
codes into the exceptions of ``theano_quantize.errors``.  There is no CPU
fallback: if the library is missing, loading fails loudly.
"""
from __future__ import annotations

import ctypes
import os

from .errors import raise_for_status

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(PKG_DIR, "libtq.so")

_i64 = ctypes.c_int64
_int = ctypes.c_int
_dbl = ctypes.c_double
_p = ctypes.c_void_p

# name -> argtypes (all return int status unless listed in _RESTYPE)
SIGNATURES = {
    "tq_version": [],
    "tq_status_string": [_int],
    "tq_last_error": [],
    "tq_qdtype_info": [_int, _p, _p, _p, _p],
    "tq_quantize_tensor": [_p, _i64, _dbl, _dbl, _int, _p, _p],
    "tq_dequantize_tensor": [_p, _i64, _dbl, _dbl, _p, _p],
    "tq_fake_quantize": [_p, _i64, _dbl, _dbl, _int, _p, _p],
    "tq_quantize_per_tensor": [_p, _i64, _int, _p, _p, _p, _p],
    "tq_minmax_reset": [_p, _i64, _p],
    "tq_minmax_observe": [_p, _i64, _p, _p],
    "tq_minmax_observe_per_channel": [_p, _i64, _i64, _p, _p],
    "tq_quantize_tensor_f64": [_p, _i64, _dbl, _dbl, _int, _p, _p],
    "tq_dequantize_tensor_f64": [_p, _i64, _dbl, _dbl, _p, _p],
    "tq_fake_quantize_f64": [_p, _i64, _dbl, _dbl, _int, _p, _p],
    "tq_quantize_per_tensor_f64": [_p, _i64, _int, _p, _p, _p, _p],
    "tq_minmax_reset_f64": [_p, _i64, _p],
    "tq_minmax_observe_f64": [_p, _i64, _p, _p],
    "tq_minmax_observe_per_channel_f64": [_p, _i64, _i64, _p, _p],
    "tq_observer_scale_zp": [_dbl, _dbl, _int, _int, _p, _p],
    "tq_quantize_i8_rowwise": [_p, _i64, _i64, _p, _p, _p],
    "tq_dequantize_i8_rowwise": [_p, _p, _i64, _i64, _p, _p],
    "tq_fake_quantize_i8_rowwise": [_p, _i64, _i64, _p, _p, _p, _p],
    "tq_quantize_fp8_rowwise": [_p, _i64, _i64, _p, _p, _p],
    "tq_dequantize_fp8_rowwise": [_p, _p, _i64, _i64, _p, _p],
    "tq_fake_quantize_fp8_rowwise": [_p, _i64, _i64, _p, _p, _p, _p],
    "tq_quantize_i4_g128": [_p, _i64, _i64, _p, _p, _p],
    "tq_dequantize_i4_g128": [_p, _p, _i64, _i64, _p, _p],
    "tq_gemv_w8": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_gemv_fp8": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_gemv_w8a8": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_gemv_fp8a8": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_gemv_w4g128": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_w4g128_tile_rows": [_i64],
    "tq_repack_w4g128_tiled": [_p, _p, _i64, _i64, _i64, _p, _p, _p],
    "tq_gemv_w4g128_tiled": [_p, _i64, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "tq_gemm_w8a8": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p, _p],
    "tq_gemm_fp8": [_p, _p, _p, _p, _p, _i64, _i64, _i64, _p, _p],
    "tq_dtype_size": [_int],
    "tq_convert": [_p, _int, _p, _int, _i64, _p],
    "tq_attention_f32": [_p, _i64, _p, _i64, _p, _i64, _p, _i64, _i64, _i64, _i64, _i64, _p, _i64, _p],
    "tq_gemm_w4g128_bf16": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _p],
    "tq_gemm_w4g128_bf16_workspace_bytes": [_i64, _i64],
    "tq_gemm_w4g128_bf16_ws": [_p, _i64, _p, _p, _p, _i64, _i64, _p, _i64, _p, _p],
    "tq_mlp_w4g128_workspace_bytes": [_i64, _i64, _i64],
    "tq_mlp_w4g128": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p, _p, _i64, _p, _p],
    "tq_mlp_w4g128_decode_workspace_bytes": [_i64, _i64, _i64],
    "tq_repack_w4g128_gate_up_tiled": [_p, _p, _p, _p, _i64, _i64, _p, _p, _p],
    "tq_mlp_w4g128_decode": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p, _i64, _p, _p],
    "tq_mlp_w4g128_decode_noalloc": [_p, _i64, _i64, _i64, _p, _p, _p, _p, _i64, _p, _p],
}
_RESTYPE = {"tq_status_string": ctypes.c_char_p, "tq_last_error": ctypes.c_char_p,
            "tq_w4g128_tile_rows": ctypes.c_int64, "tq_mlp_w4g128_workspace_bytes": ctypes.c_int64,
            "tq_mlp_w4g128_decode_workspace_bytes": ctypes.c_int64,
            "tq_gemm_w4g128_bf16_workspace_bytes": ctypes.c_int64, "tq_dtype_size": ctypes.c_int64}

_lib = None


def lib():
    """Loads libtq.so once and returns the ctypes handle."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"libtq.so is not built ({LIB_PATH}); run `python neo-theano_amd/build.py`")
        L = ctypes.CDLL(LIB_PATH)
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, _int)
        _lib = L
    return _lib


def call(name, *args):
    """Calls a status-returning entry point and raises the mapped exception."""
    L = lib()
    st = getattr(L, name)(*args)
    if st != 0:
        msg = L.tq_last_error().decode(errors="replace")
        raise_for_status(st, f"{name}: {msg}")
    return st
