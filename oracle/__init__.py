"""ctypes view of the C oracle (oracle/tq_oracle.c).

TEST INFRASTRUCTURE ONLY: the parity checker.  Only tests/, the smoke check in
__graft_entry__.py and bench.py's cpu_baseline leg may import this module, and
only to check or to time the CPU restatement of the reference -- never as a
product path.  The library is built by ``build_oracle()`` in neo-theano_amd/build.py.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TQ_ORACLE_LIB selects another build of the same source (the sanitizer build
# of `neo-theano_amd/build.py --sanitize`)
LIB_PATH = os.environ.get("TQ_ORACLE_LIB") or os.path.join(HERE, "libtq_oracle.so")

INT8, UINT8, INT4, FP8 = 0, 1, 2, 3

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        i64, d, p = ctypes.c_int64, ctypes.c_double, ctypes.c_void_p
        sig = {
            "tqo_bits": ([ctypes.c_int], ctypes.c_int),
            "tqo_is_signed": ([ctypes.c_int], ctypes.c_int),
            "tqo_qmin": ([ctypes.c_int], d),
            "tqo_qmax": ([ctypes.c_int], d),
            "tqo_quantize_tensor": ([p, i64, d, d, ctypes.c_int, p], None),
            "tqo_dequantize_tensor": ([p, i64, d, d, p], None),
            "tqo_quantize_per_tensor": ([p, i64, ctypes.c_int, p, p, p], None),
            "tqo_fake_quantize": ([p, i64, d, d, ctypes.c_int, p], None),
            "tqo_minmax_observe": ([p, p, i64], None),
            "tqo_minmax_scale_zp": ([p, ctypes.c_int, p, p], None),
            "tqo_perchannel_observe": ([p, p, i64, p, i64], None),
            "tqo_perchannel_scales_zps": ([p, p, i64, ctypes.c_int, p, p], None),
            "tqo_perchannel_global_scale_zp": ([p, p, i64, ctypes.c_int, p, p], None),
            "tqo_mm": ([p, p, i64, i64, i64, p], None),
            "tqo_linear": ([p, i64, p, p, i64, i64, p], None),
            "tqo_sigmoid": ([d], d),
            "tqo_silu_module": ([d], d),
            "tqo_f64_to_f16_bits": ([d], ctypes.c_uint16),
            "tqo_f16_bits_to_f64": ([ctypes.c_uint16], d),
            "tqo_f32_to_bf16_bits": ([ctypes.c_float], ctypes.c_uint16),
            "tqo_bf16_bits_to_f64": ([ctypes.c_uint16], d),
            "tqo_quantize_i8_rowwise": ([p, i64, i64, p, p], None),
            "tqo_dequantize_i8_rowwise": ([p, p, i64, i64, p], None),
            "tqo_quantize_i4_g128": ([p, i64, i64, p, p], None),
            "tqo_dequantize_i4_g128": ([p, p, i64, i64, p], None),
            "tqo_linear_w8": ([p, i64, p, p, p, i64, i64, p], None),
            "tqo_linear_w4g128_bf16": ([p, i64, p, p, p, i64, i64, p], None),
            "tqo_linear_w4g128_f32": ([p, i64, p, p, p, i64, i64, p], None),
            "tqo_gemm_w8a8_acc": ([p, p, i64, i64, i64, p], None),
            "tqo_linear_w8a8": ([p, p, p, p, p, i64, i64, i64, p], None),
            "tqo_mlp_w4g128": ([p, i64, i64, i64, p, p, p, p, p, p, p], None),
            "tqo_e4m3_to_f64": ([ctypes.c_uint8], d),
            "tqo_f64_to_bf16_bits": ([d], ctypes.c_uint16),
            "tqo_dtype_size": ([ctypes.c_int], i64),
            "tqo_convert": ([p, ctypes.c_int, p, ctypes.c_int, i64], None),
            "tqo_attention": ([p, p, p, p, i64, i64, i64, i64, i64, p], None),
            "tqo_f32_to_e4m3": ([ctypes.c_float], ctypes.c_uint8),
            "tqo_quantize_fp8_rowwise": ([p, i64, i64, p, p], None),
            "tqo_dequantize_fp8_rowwise": ([p, p, i64, i64, p], None),
            "tqo_linear_fp8": ([p, p, p, p, p, i64, i64, i64, p], None),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- reference primitives (f64 in / f64 out) ----

def quantize_tensor(x, scale, zero_point, dtype):
    x = _c(x, np.float64)
    q = np.empty_like(x)
    lib().tqo_quantize_tensor(_ptr(x), x.size, float(scale), float(zero_point), dtype, _ptr(q))
    return q


def dequantize_tensor(q, scale, zero_point):
    q = _c(q, np.float64)
    out = np.empty_like(q)
    lib().tqo_dequantize_tensor(_ptr(q), q.size, float(scale), float(zero_point), _ptr(out))
    return out


def quantize_per_tensor(x, dtype):
    x = _c(x, np.float64)
    q = np.empty_like(x)
    s = np.zeros(1)
    z = np.zeros(1)
    lib().tqo_quantize_per_tensor(_ptr(x), x.size, dtype, _ptr(q), _ptr(s), _ptr(z))
    return q, float(s[0]), float(z[0])


def fake_quantize(x, scale, zero_point, dtype):
    x = _c(x, np.float64)
    out = np.empty_like(x)
    lib().tqo_fake_quantize(_ptr(x), x.size, float(scale), float(zero_point), dtype, _ptr(out))
    return out


class MinMaxObserver:
    def __init__(self):
        self.state = np.array([np.inf, -np.inf, 0.0])

    def observe(self, values):
        v = _c(values, np.float64)
        lib().tqo_minmax_observe(_ptr(self.state), _ptr(v), v.size)

    def compute_scale_zero_point(self, dtype):
        s = np.zeros(1)
        z = np.zeros(1)
        lib().tqo_minmax_scale_zp(_ptr(self.state), dtype, _ptr(s), _ptr(z))
        return float(s[0]), float(z[0])

    def reset(self):
        self.state[:] = [np.inf, -np.inf, 0.0]

    @property
    def min_val(self):
        return float(self.state[0])

    @property
    def max_val(self):
        return float(self.state[1])


class PerChannelMinMaxObserver:
    def __init__(self, channels):
        self.channels = channels
        self.mins = np.full(channels, np.inf)
        self.maxs = np.full(channels, -np.inf)

    def observe(self, values):
        v = _c(values, np.float64)
        lib().tqo_perchannel_observe(_ptr(self.mins), _ptr(self.maxs), self.channels, _ptr(v), v.size)

    def scales_and_zero_points(self, dtype):
        s = np.zeros(self.channels)
        z = np.zeros(self.channels)
        lib().tqo_perchannel_scales_zps(_ptr(self.mins), _ptr(self.maxs), self.channels, dtype,
                                        _ptr(s), _ptr(z))
        return s, z

    def compute_scale_zero_point(self, dtype):
        s = np.zeros(1)
        z = np.zeros(1)
        lib().tqo_perchannel_global_scale_zp(_ptr(self.mins), _ptr(self.maxs), self.channels,
                                             dtype, _ptr(s), _ptr(z))
        return float(s[0]), float(z[0])

    def reset(self):
        self.mins[:] = np.inf
        self.maxs[:] = -np.inf


def mm(a, b):
    a = _c(a, np.float64)
    b = _c(b, np.float64)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n))
    lib().tqo_mm(_ptr(a), _ptr(b), m, k, n, _ptr(c))
    return c


def linear(x, w, bias=None):
    x = _c(x, np.float64)
    w = _c(w, np.float64)
    b = None if bias is None else _c(bias, np.float32)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear(_ptr(x), m, _ptr(w), _ptr(b), n, k, _ptr(y))
    return y


def sigmoid(x):
    return lib().tqo_sigmoid(float(x))


def silu_module(x):
    return lib().tqo_silu_module(float(x))


def f64_to_f16_bits(x):
    return lib().tqo_f64_to_f16_bits(float(x))


def f16_bits_to_f64(h):
    return lib().tqo_f16_bits_to_f64(int(h))


def f32_to_bf16_bits(x):
    return lib().tqo_f32_to_bf16_bits(float(x))


def bf16_bits_to_f64(b):
    return lib().tqo_bf16_bits_to_f64(int(b))


# ---- build-defined compositions (f32 / packed in, bit-exact outputs) ----

def quantize_i8_rowwise(w):
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.int8)
    s = np.empty(n, np.float32)
    lib().tqo_quantize_i8_rowwise(_ptr(w), n, k, _ptr(q), _ptr(s))
    return q, s


def dequantize_i8_rowwise(q, s):
    q = _c(q, np.int8)
    s = _c(s, np.float32)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().tqo_dequantize_i8_rowwise(_ptr(q), _ptr(s), n, k, _ptr(out))
    return out


def quantize_i4_g128(w):
    w = _c(w, np.float32)
    n, k = w.shape
    assert k % 128 == 0
    p = np.empty((n, k // 2), np.uint8)
    s = np.empty((n, k // 128), np.uint16)
    lib().tqo_quantize_i4_g128(_ptr(w), n, k, _ptr(p), _ptr(s))
    return p, s


def dequantize_i4_g128(p, s):
    p = _c(p, np.uint8)
    s = _c(s, np.uint16)
    n, kh = p.shape
    out = np.empty((n, kh * 2), np.float32)
    lib().tqo_dequantize_i4_g128(_ptr(p), _ptr(s), n, kh * 2, _ptr(out))
    return out


def linear_w8(x, q, s, bias=None):
    x = _c(x, np.float32)
    q = _c(q, np.int8)
    s = _c(s, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    m, k = x.shape
    n = q.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear_w8(_ptr(x), m, _ptr(q), _ptr(s), _ptr(b), n, k, _ptr(y))
    return y


def linear_w4g128_bf16(x_bf16_bits, p, s, bias=None):
    x = _c(x_bf16_bits, np.uint16)
    p = _c(p, np.uint8)
    s = _c(s, np.uint16)
    b = None if bias is None else _c(bias, np.float32)
    m, k = x.shape
    n = p.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear_w4g128_bf16(_ptr(x), m, _ptr(p), _ptr(s), _ptr(b), n, k, _ptr(y))
    return y


def linear_w4g128_f32(x, p, s, bias=None):
    x = _c(x, np.float32)
    p = _c(p, np.uint8)
    s = _c(s, np.uint16)
    b = None if bias is None else _c(bias, np.float32)
    m, k = x.shape
    n = p.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear_w4g128_f32(_ptr(x), m, _ptr(p), _ptr(s), _ptr(b), n, k, _ptr(y))
    return y


def gemm_w8a8_acc(qa, qw):
    qa = _c(qa, np.int8)
    qw = _c(qw, np.int8)
    m, k = qa.shape
    n = qw.shape[0]
    acc = np.empty((m, n), np.int32)
    lib().tqo_gemm_w8a8_acc(_ptr(qa), _ptr(qw), m, n, k, _ptr(acc))
    return acc


def linear_w8a8(qa, sa, qw, sw, bias=None):
    qa = _c(qa, np.int8)
    qw = _c(qw, np.int8)
    sa = _c(sa, np.float32)
    sw = _c(sw, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    m, k = qa.shape
    n = qw.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear_w8a8(_ptr(qa), _ptr(sa), _ptr(qw), _ptr(sw), _ptr(b), m, n, k, _ptr(y))
    return y


def mlp_w4g128(x_bf16_bits, pg, sg, pu, su, pd, sd):
    x = _c(x_bf16_bits, np.uint16)
    m, d = x.shape
    f = pg.shape[0]
    args = [_c(pg, np.uint8), _c(sg, np.uint16), _c(pu, np.uint8), _c(su, np.uint16),
            _c(pd, np.uint8), _c(sd, np.uint16)]
    y = np.empty((m, d))
    lib().tqo_mlp_w4g128(_ptr(x), m, d, f, *[_ptr(a) for a in args], _ptr(y))
    return y


# ---- build-defined FP8 (OCP e4m3) ----

def e4m3_to_f64(b):
    return lib().tqo_e4m3_to_f64(int(b))


def f32_to_e4m3(x):
    return lib().tqo_f32_to_e4m3(float(x))


def quantize_fp8_rowwise(w):
    w = _c(w, np.float32)
    n, k = w.shape
    q = np.empty((n, k), np.uint8)
    s = np.empty(n, np.float32)
    lib().tqo_quantize_fp8_rowwise(_ptr(w), n, k, _ptr(q), _ptr(s))
    return q, s


def dequantize_fp8_rowwise(q, s):
    q = _c(q, np.uint8)
    s = _c(s, np.float32)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    lib().tqo_dequantize_fp8_rowwise(_ptr(q), _ptr(s), n, k, _ptr(out))
    return out


def linear_fp8(qa, sa, qw, sw, bias=None):
    qa = _c(qa, np.uint8)
    qw = _c(qw, np.uint8)
    sa = _c(sa, np.float32)
    sw = _c(sw, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    m, k = qa.shape
    n = qw.shape[0]
    y = np.empty((m, n))
    lib().tqo_linear_fp8(_ptr(qa), _ptr(sa), _ptr(qw), _ptr(sw), _ptr(b), m, n, k, _ptr(y))
    return y


# ---- element conversion (DType order) ----
DTYPES = ["float16", "bfloat16", "float32", "float64", "uint8", "int8", "int16", "int32", "int64", "bool"]
NP_STORAGE = [np.uint16, np.uint16, np.float32, np.float64, np.uint8, np.int8, np.int16, np.int32, np.int64, np.uint8]


def f64_to_bf16_bits(x):
    return lib().tqo_f64_to_bf16_bits(float(x))


def convert(src, src_t, dst_t):
    """src: numpy array in the storage type of src_t (F16/BF16 as uint16 bits,
    Bool as uint8) -> numpy array in the storage type of dst_t."""
    src = _c(src, NP_STORAGE[src_t])
    out = np.empty(src.shape, NP_STORAGE[dst_t])
    lib().tqo_convert(_ptr(src), src_t, _ptr(out), dst_t, src.size)
    return out


# ---- attention core (transformer.rs:95-142) ----

def attention(q, k, v, heads, mask=None):
    """q, k, v: [B, S, E] f64 -> [B, S, E] f64; mask None or [Bm, S, S] (Bm 1 or B)."""
    q = _c(q, np.float64)
    k = _c(k, np.float64)
    v = _c(v, np.float64)
    B, S, E = q.shape
    m = None if mask is None else _c(mask, np.float64)
    out = np.empty((B, S, E))
    lib().tqo_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(m), 0 if m is None else m.shape[0], B, S, heads,
                        E // heads, _ptr(out))
    return out
