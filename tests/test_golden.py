"""Golden fixtures (tests/golden/) checked on the CPU.

* reference_kats.json holds the values the reference's own unit tests assert
  (each case names its file:line); the oracle must reproduce them.
* The .npz cases freeze the oracle's outputs for the build-defined formats and
  the synthetic-data generator; the oracle and the generator must reproduce
  them byte for byte.  The GPU kernels are checked against the same files in
  test_gpu_golden.py.
"""
import json
import os

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
DT = {"Int8": 0, "UInt8": 1, "Int4": 2, "FP8": 3}


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def as_f64(v):
    return np.array([float(t) for t in v], dtype=np.float64)


def test_kat_qdtype_ranges(oracle):
    for c in kats()["qdtype_ranges"]["cases"]:
        d = DT[c["dtype"]]
        lib = oracle.lib()
        assert lib.tqo_bits(d) == c["bits"]
        assert bool(lib.tqo_is_signed(d)) == c["signed"]
        assert lib.tqo_qmin(d) == c["qmin"] and lib.tqo_qmax(d) == c["qmax"]


def test_kat_quantize_tensor(oracle):
    for c in kats()["quantize_tensor"]["cases"]:
        q = oracle.quantize_tensor(as_f64(c["x"]), c["scale"], c["zp"], DT[c["dtype"]])
        want = as_f64(c["q"])
        assert np.array_equal(q, want), (c, q)
        assert np.array_equal(np.signbit(q), np.signbit(want)), (c, q)  # -0.0 kept


def test_kat_dequantize_tensor(oracle):
    for c in kats()["dequantize_tensor"]["cases"]:
        x = oracle.dequantize_tensor(as_f64(c["q"]), c["scale"], c["zp"])
        assert np.all(np.abs(x - as_f64(c["x"])) < c["tol"])


def test_kat_quantize_per_tensor(oracle):
    for c in kats()["quantize_per_tensor_roundtrip"]["cases"]:
        x = as_f64(c["x"])
        q, s, z = oracle.quantize_per_tensor(x, DT[c["dtype"]])
        assert np.all(np.abs(oracle.dequantize_tensor(q, s, z) - x) < c["tol"])
    for c in kats()["quantize_per_tensor_range"]["cases"]:
        q, _, _ = oracle.quantize_per_tensor(as_f64(c["x"]), DT[c["dtype"]])
        assert np.all((q >= c["lo"]) & (q <= c["hi"]))


def test_kat_minmax_observer(oracle):
    for c in kats()["minmax_observer"]["cases"]:
        obs = oracle.MinMaxObserver()
        for v in c["observe"]:
            obs.observe(as_f64(v))
        if "min" in c:
            assert obs.min_val == c["min"] and obs.max_val == c["max"]
        if "scale" in c:
            s, z = obs.compute_scale_zero_point(DT[c["dtype"]])
            tol = c.get("tol", 0.0)
            assert abs(s - c["scale"]) <= tol
            if tol == 0.0:
                assert z == c["zp"]


def test_kat_matmul(oracle):
    for c in kats()["matmul"]["cases"]:
        got = oracle.mm(np.array(c["a"], np.float64), np.array(c["b"], np.float64))
        assert np.array_equal(got, np.array(c["c"], np.float64))


def test_kat_sigmoid(oracle):
    for c in kats()["sigmoid"]["cases"]:
        assert abs(oracle.sigmoid(c["x"]) - c["y"]) < c["tol"]


def test_fixture_int8_rowwise(oracle):
    d = load("int8_rowwise_64x256.npz")
    q, s = oracle.quantize_i8_rowwise(d["w"])
    assert np.array_equal(q, d["q"]) and np.array_equal(s.view(np.uint32), d["s"].view(np.uint32))
    assert np.array_equal(oracle.dequantize_i8_rowwise(q, s).view(np.uint32), d["w_hat"].view(np.uint32))
    # edge rows: zero row -> floor scale, +-1 row -> codes +-127
    assert d["s"][0] == np.float32(1e-10) and np.all(d["q"][0] == 0)
    assert set(np.unique(d["q"][2])) == {-127, 127}


def test_fixture_int4_g128(oracle):
    d = load("int4_g128_16x256.npz")
    p, s = oracle.quantize_i4_g128(d["w"])
    assert np.array_equal(p, d["packed"]) and np.array_equal(s, d["s_f16"])
    assert np.array_equal(oracle.dequantize_i4_g128(p, s).view(np.uint32), d["w_hat"].view(np.uint32))
    assert d["s_f16"][0, 0] == 1          # 2^-24 floor for the zero group
    assert d["s_f16"][1, 1] == 0x3C00     # absmax 7 -> scale 1.0


def test_fixture_w8a8(oracle):
    d = load("w8a8_4x256x8.npz")
    qa, sa = oracle.quantize_i8_rowwise(d["x"])
    qw, sw = oracle.quantize_i8_rowwise(d["w"])
    assert np.array_equal(qa, d["qa"]) and np.array_equal(qw, d["qw"])
    acc = oracle.gemm_w8a8_acc(qa, qw)
    assert np.array_equal(acc, d["acc"])
    # int64 brute force of the same accumulators (independent of the oracle)
    assert np.array_equal(d["qa"].astype(np.int64) @ d["qw"].astype(np.int64).T, d["acc"])
    assert np.array_equal(oracle.linear_w8a8(qa, sa, qw, sw), d["y"])


def test_fixture_synth_prefixes():
    from theano_quantize import synth

    d = load("synth_prefixes.npz")
    for name, seed in synth.SEEDS.items():
        for stream in (0, 1, 2):
            v = synth.normal_f32(seed, (16,), 1.0, stream=stream)
            assert np.array_equal(v.view(np.uint32), d[f"{name}_s{stream}"]), (name, stream)
