"""GPU kernels against the golden fixtures (tests/golden/): the reference's own
known answers and the frozen oracle outputs of the build-defined formats."""
import json
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def kats():
    with open(os.path.join(GOLDEN, "reference_kats.json")) as f:
        return json.load(f)


def load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def dt(tq, name):
    return getattr(tq.QuantDType, name)


def test_kat_quantize_tensor_gpu(tq):
    for c in kats()["quantize_tensor"]["cases"]:
        x = np.array([float(v) for v in c["x"]], np.float32)
        q = tq.quantize_tensor(x, c["scale"], c["zp"], dt(tq, c["dtype"])).cpu().numpy().astype(np.float64)
        want = np.array([float(v) for v in c["q"]], np.float64)
        assert np.array_equal(q, want) and np.array_equal(np.signbit(q), np.signbit(want)), (c, q)


def test_kat_dequantize_and_per_tensor_gpu(tq):
    for c in kats()["dequantize_tensor"]["cases"]:
        x = tq.dequantize_tensor(np.array(c["q"], np.float32), c["scale"], c["zp"]).cpu().numpy()
        # f32 result of the f64 product: within one f32 ulp of the asserted values
        assert np.all(np.abs(x - np.array(c["x"])) <= np.spacing(np.float32(1.27)))
    for c in kats()["quantize_per_tensor_roundtrip"]["cases"]:
        x = np.array(c["x"], np.float32)
        q, s, z = tq.quantize_per_tensor(x, dt(tq, c["dtype"]))
        back = tq.dequantize_tensor(q, s, z).cpu().numpy()
        assert np.all(np.abs(back - x) < c["tol"])
    for c in kats()["quantize_per_tensor_range"]["cases"]:
        q, _, _ = tq.quantize_per_tensor(np.array(c["x"], np.float32), dt(tq, c["dtype"]))
        q = q.cpu().numpy()
        assert np.all((q >= c["lo"]) & (q <= c["hi"]))


def test_kat_minmax_observer_gpu(tq):
    for c in kats()["minmax_observer"]["cases"]:
        obs = tq.MinMaxObserver()
        for v in c["observe"]:
            obs.observe(np.array(v, np.float32))
        if "min" in c:
            assert obs.min_val() == c["min"] and obs.max_val() == c["max"]
        if "scale" in c:
            s, z = obs.compute_scale_zero_point(dt(tq, c["dtype"]))
            tol = c.get("tol", 0.0)
            assert abs(s - c["scale"]) <= tol
            if tol == 0.0:
                assert z == c["zp"]


def test_fixture_int8_rowwise_gpu(tq):
    d = load("int8_rowwise_64x256.npz")
    q, s = tq.quantize_per_channel_i8(d["w"])
    assert np.array_equal(q.cpu().numpy(), d["q"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), d["s"].view(np.uint32))
    w_hat = tq.dequantize_per_channel_i8(q, s).cpu().numpy()
    assert np.array_equal(w_hat.view(np.uint32), d["w_hat"].view(np.uint32))


def test_fixture_int4_g128_gpu(tq):
    d = load("int4_g128_16x256.npz")
    p, s = tq.quantize_i4_g128(d["w"])
    assert np.array_equal(p.cpu().numpy(), d["packed"])
    assert np.array_equal(s.cpu().numpy().view(np.uint16), d["s_f16"])
    w_hat = tq.dequantize_i4_g128(p, s).cpu().numpy()
    assert np.array_equal(w_hat.view(np.uint32), d["w_hat"].view(np.uint32))


def test_fixture_w8a8_gpu(tq):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    d = load("w8a8_4x256x8.npz")
    qa, sa = tq.quantize_per_channel_i8(d["x"])
    qw, sw = tq.quantize_per_channel_i8(d["w"])
    assert np.array_equal(qa.cpu().numpy(), d["qa"]) and np.array_equal(qw.cpu().numpy(), d["qw"])
    m, k = d["x"].shape
    n = d["w"].shape[0]
    # N = 8 is below the kernel tile's 16-row granularity: pad the weight rows
    qw16 = torch.zeros((16, k), dtype=torch.int8, device="cuda")
    qw16[:n] = qw
    sw16 = torch.ones(16, dtype=torch.float32, device="cuda")
    sw16[:n] = sw
    acc = torch.empty((m, 16), dtype=torch.int32, device="cuda")
    y = torch.empty((m, 16), dtype=torch.float32, device="cuda")
    _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(qw16), ptr(sw16), None, m, 16, k, ptr(acc), ptr(y), stream())
    torch.cuda.synchronize()
    assert np.array_equal(acc.cpu().numpy()[:, :n], d["acc"])
    got = y.cpu().numpy()[:, :n].astype(np.float64)
    assert np.all(np.abs(got - d["y"]) <= 1e-4 + 1e-3 * np.abs(d["y"]))
