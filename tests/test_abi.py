"""CPU checks of the C ABI: libtq.so loads, exports every entry point that
include/tq.h declares, and its host-only paths (ranges, observer scale math,
argument validation) behave like the reference.  No kernel is launched here:
every call below fails validation or is host-only."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tq.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\**(tq_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def abi():
    from theano_quantize import _abi

    return _abi


def test_header_declares_entry_points():
    syms = declared_symbols()
    assert "tq_quantize_i8_rowwise" in syms and "tq_gemm_w8a8" in syms and len(syms) >= 20


def test_library_exports_every_declared_symbol(abi):
    L = abi.lib()
    missing = [s for s in declared_symbols() if not hasattr(L, s)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol(abi):
    assert sorted(abi.SIGNATURES) == declared_symbols()


def test_version_and_status_strings(abi):
    L = abi.lib()
    assert L.tq_version() >= 100
    assert L.tq_status_string(0) == b"TQ_OK" and L.tq_status_string(1) == b"TQ_EINVAL"


def test_qdtype_info_reference_ranges(abi):
    # crates/theano-quantize/src/qconfig.rs:82-108
    from theano_quantize import QuantDType

    assert [d.bits() for d in QuantDType] == [8, 8, 4, 8]
    assert [d.is_signed() for d in QuantDType] == [True, False, True, False]
    assert [d.qmin() for d in QuantDType] == [-128.0, 0.0, -8.0, -448.0]
    assert [d.qmax() for d in QuantDType] == [127.0, 255.0, 7.0, 448.0]
    with pytest.raises(ValueError):
        abi.call("tq_qdtype_info", 9, None, None, None, None)


def test_qconfig_defaults_reference():
    # qconfig.rs:110-148
    from theano_quantize import QConfig, QuantDType

    c = QConfig.default_int8()
    assert (c.weight_dtype, c.activation_dtype, c.symmetric, c.per_channel) == (
        QuantDType.Int8, QuantDType.UInt8, True, False)
    c = QConfig.default_int4()
    assert (c.weight_dtype, c.activation_dtype, c.symmetric, c.per_channel) == (
        QuantDType.Int4, QuantDType.Int8, True, True)
    assert QConfig.default() == QConfig.default_int8()


def test_observer_scale_zp_matches_oracle(abi, oracle):
    s, z = ctypes.c_double(), ctypes.c_double()
    for mn, mx, dt in [(-1.0, 3.0, 0), (0.0, 1.0, 1), (-0.2, 0.7, 2), (5.0, 5.0, 0),
                       (float("inf"), float("-inf"), 0), (-448.0, 100.0, 3)]:
        abi.call("tq_observer_scale_zp", mn, mx, 1, dt, ctypes.byref(s), ctypes.byref(z))
        o = oracle.MinMaxObserver()
        o.state[:] = [mn, mx, 1.0]
        assert (s.value, z.value) == o.compute_scale_zero_point(dt)
    abi.call("tq_observer_scale_zp", 0.0, 1.0, 0, 0, ctypes.byref(s), ctypes.byref(z))
    assert (s.value, z.value) == (1.0, 0.0)  # uninitialized, observer.rs:52-54


@pytest.mark.parametrize("call", [
    ("tq_quantize_i4_g128", [None, 4, 100, None, None, None]),            # K % 128
    ("tq_dequantize_i4_g128", [None, None, 2, 130, None, None]),
    ("tq_quantize_i8_rowwise", [None, -1, 16, None, None, None]),         # negative rows
    ("tq_quantize_i8_rowwise", [None, 4, 16, None, None, None]),          # null pointers
    ("tq_gemv_w4g128", [None, 17, None, None, None, 16, 128, None, None]),  # M > 16
    ("tq_gemv_w8", [None, 1, None, None, None, 16, 20, None, None]),       # K % 16
    ("tq_gemm_w8a8", [None, None, None, None, None, 4, 20, 64, None, None, None]),  # N % 16
    ("tq_gemm_w8a8", [None, None, None, None, None, 4, 16, 65, None, None, None]),  # K % 16
    ("tq_gemm_w4g128_bf16", [None, 4, None, None, None, 16, 100, None, None]),
    ("tq_mlp_w4g128", [None, 4, 100, 128, None, None, None, None, None, None, None, 0, None, None]),  # D % 128
    ("tq_mlp_w4g128", [None, 4, 256, 256, None, None, None, None, None, None, None, 0, None, None]),  # nulls
    ("tq_mlp_w4g128", [256, 4, 256, 256, 256, 256, 256, 256, 256, 256, 256, 16, 256, None]),  # workspace
    ("tq_mlp_w4g128_decode", [None, 17, 256, 256, None, None, None, None, 16, None, 0, None, None]),  # M > 16
    ("tq_mlp_w4g128_decode", [None, 2, 100, 256, None, None, None, None, 16, None, 0, None, None]),  # D % 128
    ("tq_mlp_w4g128_decode", [None, 2, 256, 32768, None, None, None, None, 16, None, 0, None, None]),  # F > 16384
    ("tq_mlp_w4g128_decode", [None, 2, 256, 256, None, None, None, None, 24, None, 0, None, None]),  # tile rows
    ("tq_mlp_w4g128_decode", [None, 2, 256, 256, None, None, None, None, 16, None, 0, None, None]),  # nulls
    ("tq_mlp_w4g128_decode", [256, 2, 256, 256, 256, 256, 256, 256, 16, 256, 16, 256, None]),  # workspace
    ("tq_mlp_w4g128_decode_noalloc", [256, 17, 256, 16384, 256, 256, 256, 256, 16, 256, None]),  # scratch
    ("tq_mlp_w4g128_decode_noalloc", [256, 16, 256, 16512, 256, 256, 256, 256, 16, 256, None]),  # scratch
    ("tq_mlp_w4g128_decode_noalloc", [256, 2, 256, 256, 256, 256, 256, 256, 16, None, None]),  # null y
    ("tq_repack_w4g128_gate_up_tiled", [None, None, None, None, 128, 100, None, None, None]),  # D % 128
    ("tq_repack_w4g128_gate_up_tiled", [None, None, None, None, 128, 128, None, None, None]),  # nulls
    ("tq_quantize_tensor", [None, 10, 1.0, 0.0, 7, None, None]),          # bad QuantDType
    ("tq_quantize_per_tensor", [None, 10, 0, None, None, None, None]),
    ("tq_minmax_reset", [None, 0, None]),
    ("tq_convert", [None, 3, None, 12, 4, None]),                          # unsupported dtype
    ("tq_convert", [None, 3, None, 2, -1, None]),                          # negative length
    ("tq_convert", [None, 3, None, 2, 4, None]),                           # null pointers
    ("tq_quantize_fp8_rowwise", [None, 4, 16, None, None, None]),         # null pointers
    ("tq_gemm_fp8", [None, None, None, None, None, -1, 16, 128, None, None]),  # negative shape
    ("tq_gemv_fp8", [None, 17, None, None, None, 16, 128, None, None]),   # M > 16
    ("tq_gemv_w8a8", [16, 1, 16, 16, None, 16, 100, 16, None]),           # K % 16 (fused path)
    ("tq_gemv_fp8a8", [16, 17, 16, 16, None, 16, 128, 16, None]),         # M > 16
    ("tq_attention_f32", [16, 8, 16, 8, 16, 8, None, 0, 1, 4, 2, 200, 16, 8, None]),  # head_dim > 128
])
def test_invalid_arguments_are_rejected(abi, call):
    from theano_quantize import InvalidArgument

    name, args = call
    with pytest.raises(InvalidArgument):
        abi.call(name, *args)
    assert abi.lib().tq_last_error()  # a message was recorded


def test_mlp_workspace_bytes(abi):
    ws = abi.lib().tq_mlp_w4g128_workspace_bytes
    # x in k-order (M*D*2) + x group sums (D/128 * Mpad * 8) + h hi/lo (2 * M*F*2)
    # + h group sums (F/128 * Mpad * 8), parts 256-byte aligned, Mpad = M rounded to 128
    assert ws(512, 4096, 14336) == 4194304 + 131072 + 2 * 14680064 + 458752
    m, d, f = 5, 256, 384
    parts = [m * d * 2, (d // 128) * 128 * 8, m * f * 2, m * f * 2, (f // 128) * 128 * 8]
    assert ws(m, d, f) == sum((p + 255) // 256 * 256 for p in parts)
    assert ws(1, 128, 128) >= 4 * 1 * 128  # covers the f32 h [M, F] of the shape-general path
    assert ws(0, 128, 128) == 0


def test_mlp_decode_workspace_bytes(abi):
    ws = abi.lib().tq_mlp_w4g128_decode_workspace_bytes
    # bf16 hi and lo rows of h for each token, then the f32 sums of their
    # 32-column blocks, each part rounded up to 256 bytes
    assert ws(1, 4096, 14336) == 2 * 14336 * 2 + 2 * 448 * 4
    assert ws(3, 256, 384) == 2 * 3 * 384 * 2 + 512
    assert ws(1, 128, 128) == 512 + 256
    assert ws(0, 128, 128) == 0 and ws(-1, 128, 128) == -1


def test_dtype_sizes(abi, oracle):
    # DType::size_in_bytes (crates/theano-types/src/dtype.rs:33-40) in DType order
    assert [abi.lib().tq_dtype_size(t) for t in range(10)] == [2, 2, 4, 8, 1, 1, 2, 4, 8, 1]
    assert [abi.lib().tq_dtype_size(t) for t in range(10)] == [oracle.lib().tqo_dtype_size(t) for t in range(10)]
    assert abi.lib().tq_dtype_size(10) == 0 and abi.lib().tq_dtype_size(-1) == 0


def test_zero_sizes_are_noops(abi):
    # empty inputs enqueue nothing and succeed
    assert abi.call("tq_quantize_i8_rowwise", None, 0, 16, None, None, None) == 0
    assert abi.call("tq_gemv_w8", None, 0, None, None, None, 16, 16, None, None) == 0
    assert abi.call("tq_quantize_tensor", None, 0, 1.0, 0.0, 0, None, None) == 0
    assert abi.call("tq_convert", None, 3, None, 1, 0, None) == 0


def test_host_paths_from_many_threads(abi):
    """Entry points called concurrently from 16 threads: each thread's status
    and tq_last_error message are its own (the message is thread-local), and
    the cached per-device queries agree across threads."""
    import threading

    L = abi.lib()
    cases = [
        ("tq_quantize_i4_g128", [None, 4, 100, None, None, None], b"tq_quantize_i4_g128: K=100"),
        ("tq_gemv_w4g128", [None, 17, None, None, None, 16, 128, None, None], b"tq_gemv_w4g128: M=17"),
        ("tq_convert", [None, 3, None, 12, 4, None], b"tq_convert: unsupported dtype"),
        ("tq_quantize_tensor", [None, 10, 1.0, 0.0, 7, None, None], b"unknown QuantDType 7"),
    ]
    errors, tiles = [], []

    def worker(i):
        name, args, word = cases[i % len(cases)]
        for _ in range(200):
            st = getattr(L, name)(*args)
            msg = L.tq_last_error()
            if st != 1 or not msg.startswith(word):
                errors.append((i, name, st, msg))
                return
            tiles.append(L.tq_w4g128_tile_rows(14336))
            s, z = ctypes.c_double(), ctypes.c_double()
            if L.tq_observer_scale_zp(-1.0, 3.0, 1, 0, ctypes.byref(s), ctypes.byref(z)) != 0:
                errors.append((i, "scale_zp"))
                return

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(16)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert not errors, errors[:4]
    assert len(set(tiles)) == 1


def test_python_api_rejects_non_float_data():
    import numpy as np

    import theano_quantize as tq
    from theano_quantize import InvalidArgument

    for f in (lambda x: tq.quantize_tensor(x, 1.0, 0.0, tq.QuantDType.Int8),
              lambda x: tq.dequantize_tensor(x, 1.0, 0.0),
              lambda x: tq.fake_quantize(x, 1.0, 0.0, tq.QuantDType.Int8),
              lambda x: tq.quantize_per_tensor(x, tq.QuantDType.Int8)):
        with pytest.raises(InvalidArgument):
            f(np.arange(4, dtype=np.int32))
