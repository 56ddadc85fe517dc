"""GPU parity: FP8 (OCP e4m3) per-row quantize / dequantize / fake-quantize
(bit-exact against the oracle, which is pinned to torch.float8_e4m3fn) and the
FP8 W8A8 GEMM (f32 accumulation; |got - ref| <= 1e-4 + 1e-3 * |ref| against
the oracle's f64 Linear over the dequantized operands, and at full size against
a float64 torch product of the decoded operands)."""
import numpy as np
import pytest

from conftest import assert_close, ieee_equal

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4


def dev_tensor(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def normal(seed, shape, std=1.0, stream=0):
    from theano_quantize.synth import normal_f32

    return normal_f32(seed, shape, std, stream)


def e4m3_grid():
    """Every finite e4m3 value >= 0, the ties between neighbours and their f32 neighbours."""
    import torch

    v = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn).float().numpy()
    g = np.unique(v[np.isfinite(v) & (v >= 0)])
    mids = ((g[:-1].astype(np.float64) + g[1:]) / 2).astype(np.float32)
    pts = np.concatenate([g, mids])
    pts = np.concatenate([pts, np.nextafter(pts, np.float32(np.inf)), np.nextafter(pts, np.float32(-np.inf))])
    pts = pts[np.abs(pts) <= 448.0]
    return np.concatenate([pts, -pts, np.array([-0.0, 2.0 ** -10, -(2.0 ** -10), 1e-30], np.float32)])


def test_e4m3_encode_matches_oracle_on_every_tie(tq, oracle):
    """Rows whose absmax is 448 have scale exactly 1, so the codes are the hardware
    conversion of the inputs themselves: every grid value, tie and neighbour."""
    v = e4m3_grid().astype(np.float32)
    k = 256
    pad = (-len(v)) % (k - 1)
    v = np.concatenate([v, np.zeros(pad, np.float32)]).reshape(-1, k - 1)
    w = np.concatenate([np.full((v.shape[0], 1), 448.0, np.float32), v], axis=1)
    w[0, 5] = np.nan  # NaN -> 0x7F, ignored by the scale
    q, s = tq.quantize_per_channel_fp8(dev_tensor(w))
    rq, rs = oracle.quantize_fp8_rowwise(w)
    assert np.all(rs == 1.0)
    assert np.array_equal(host(s), rs)
    assert np.array_equal(host(q), rq)
    assert host(q)[0, 5] == 0x7F


def test_e4m3_decode_all_codes(tq, oracle):
    codes = np.arange(256, dtype=np.uint8).reshape(1, 256)
    out = host(tq.dequantize_per_channel_fp8(dev_tensor(codes), dev_tensor(np.ones(1, np.float32))))
    ref = np.array([[oracle.e4m3_to_f64(c) for c in range(256)]])
    assert ieee_equal(out, ref)


@pytest.mark.parametrize("rows,k", [(3, 16), (5, 1024), (7, 1040), (4, 4096), (3, 8192), (2, 16384),
                                    (6, 100), (3, 17), (2, 20000), (0, 64)])
def test_quantize_fp8_rowwise_shapes(tq, oracle, rows, k):
    w = normal(71, (rows, k), 1.0) * np.exp2(np.arange(rows) - 3.0)[:, None].astype(np.float32)
    q, s, w_hat = tq.fake_quantize_per_channel_fp8(dev_tensor(w))
    rq, rs = oracle.quantize_fp8_rowwise(w)
    assert np.array_equal(host(q), rq) and np.array_equal(host(s), rs)
    assert ieee_equal(host(w_hat), oracle.dequantize_fp8_rowwise(rq, rs))
    q2, s2 = tq.quantize_per_channel_fp8(dev_tensor(w))
    assert np.array_equal(host(q2), rq) and np.array_equal(host(s2), rs)


@pytest.mark.parametrize("k", [64, 30, 2048, 4096])
def test_quantize_fp8_special_rows(tq, oracle, k):
    w = normal(72, (7, k), 1.0)
    w[6] *= 1e-38  # subnormal inputs
    w[1] = 0.0
    w[2, 3] = np.nan
    w[3, 4] = np.inf
    w[4, 0] = -0.0
    w[4, 1] = -1e-30
    w[5] = np.nan
    q, s, w_hat = tq.fake_quantize_per_channel_fp8(dev_tensor(w))
    rq, rs = oracle.quantize_fp8_rowwise(w)
    assert np.array_equal(host(q), rq) and ieee_equal(host(s), rs)
    assert ieee_equal(host(w_hat), oracle.dequantize_fp8_rowwise(rq, rs))


@pytest.mark.parametrize("rows,k", [(4, 4096), (3, 48), (5, 33)])
def test_dequantize_fp8_rowwise(tq, oracle, rows, k):
    rng = np.random.default_rng(73)
    q = rng.integers(0, 256, (rows, k), dtype=np.uint8)
    s = rng.uniform(0.25, 4, rows).astype(np.float32)
    out = host(tq.dequantize_per_channel_fp8(dev_tensor(q), dev_tensor(s)))
    assert ieee_equal(out, oracle.dequantize_fp8_rowwise(q, s))


# ------------------------------------------------------------------- GEMM
def run_fp8(tq, x, w, bias=None):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    m, k = x.shape
    n = w.shape[0]
    qa, sa = tq.quantize_per_channel_fp8(dev_tensor(x))
    qw, sw = tq.quantize_per_channel_fp8(dev_tensor(w))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    bd = None if bias is None else dev_tensor(bias)
    _abi.call("tq_gemm_fp8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), ptr(bd), m, n, k, ptr(y), stream())
    return qa, sa, qw, sw, y


# K % 128 == 0 with N % 16 == 0 takes the FP8 MFMA kernels: M <= 16 (K <= 8192)
# the skinny one (one to four chunks per wave, waves past K, one-block grids),
# otherwise the tiled one (1, 2, 3 and more stages; M, N tails; tile groups with
# and without the XCD remap); the rest the shape-general kernel.
@pytest.mark.parametrize("m,n,k", [(1, 16, 128), (130, 48, 256), (7, 272, 1024), (257, 128, 4096),
                                   (300, 512, 128), (129, 4096, 256), (100, 272, 384), (384, 2048, 256),
                                   (1031, 528, 512), (5, 8, 256), (33, 50, 100), (17, 16, 1000),
                                   (16, 4096, 4096), (3, 64, 8192), (16, 16, 128), (9, 1024, 384),
                                   (2, 48, 4096)])
def test_gemm_fp8_shapes_bias(tq, oracle, m, n, k):
    x = normal(74, (m, k), 1.0)
    w = normal(74, (n, k), 0.02, stream=1)
    b = normal(74, (n,), 0.1, stream=2)
    qa, sa, qw, sw, y = run_fp8(tq, x, w, b)
    rqa, rsa = oracle.quantize_fp8_rowwise(x)
    rqw, rsw = oracle.quantize_fp8_rowwise(w)
    assert np.array_equal(host(qa), rqa) and np.array_equal(host(qw), rqw)
    assert_close(host(y), oracle.linear_fp8(rqa, rsa, rqw, rsw, b), RTOL, ATOL, f"fp8 {m}x{n}x{k}")


def test_gemm_fp8_full_size_vs_torch_f64(tq, oracle):
    """M=2048, N=K=4096: sampled rows against the oracle, every row against a
    float64 torch product of the operands decoded by torch.float8_e4m3fn."""
    import torch

    x = normal(75, (2048, 4096), 1.0)
    w = normal(75, (4096, 4096), 0.02, stream=1)
    qa, sa, qw, sw, y = run_fp8(tq, x, w)
    a = qa.view(torch.float8_e4m3fn).to(torch.float64) * sa.to(torch.float64)[:, None]
    b = qw.view(torch.float8_e4m3fn).to(torch.float64) * sw.to(torch.float64)[:, None]
    ref = (a @ b.T.contiguous()).cpu().numpy()
    yh = host(y)
    assert_close(yh, ref, RTOL, ATOL, "fp8 full size vs torch f64")
    rows = np.array([0, 1, 127, 128, 1000, 2047])
    assert_close(yh[rows], oracle.linear_fp8(host(qa)[rows], host(sa)[rows], host(qw), host(sw)),
                 RTOL, ATOL, "fp8 full size sampled rows vs oracle")


@pytest.mark.parametrize("rows", [32, 16])  # the tiled and the skinny kernel
def test_gemm_fp8_extreme_codes(tq, oracle, rows):
    """Every product at +-448^2 with constant signs: |acc| = K * 448^2 (exact in f32)."""
    x = np.where(normal(76, (rows, 1024), 1.0) > 0, 448.0, -448.0).astype(np.float32)
    w = np.where(normal(76, (64, 1024), 1.0, stream=1) > 0, 448.0, -448.0).astype(np.float32)
    x[0] = 448.0
    w[0] = 448.0
    qa, sa, qw, sw, y = run_fp8(tq, x, w)
    yh = host(y)
    assert yh[0, 0] == np.float32(1024 * 448.0 * 448.0)
    assert_close(yh, oracle.linear_fp8(host(qa), host(sa), host(qw), host(sw)), RTOL, ATOL, "fp8 +-448")


def test_quantized_linear_fp8_module(tq, oracle):
    from theano_quantize import QConfig, QuantDType

    w = normal(77, (256, 512), 0.02)
    x = normal(77, (100, 512), 1.0, stream=1)
    cfg = QConfig(QuantDType.FP8, QuantDType.FP8, True, True)
    lin = tq.QuantizedLinear.from_tensors(dev_tensor(w), None, cfg)
    assert lin.mode == "fp8"
    y = host(lin(dev_tensor(x)))
    rqa, rsa = oracle.quantize_fp8_rowwise(x)
    rqw, rsw = oracle.quantize_fp8_rowwise(w)
    assert_close(y, oracle.linear_fp8(rqa, rsa, rqw, rsw), RTOL, ATOL, "QuantizedLinear fp8")


# ------------------------------------------------------------------- GEMV
@pytest.mark.parametrize("m,n,k", [(1, 14336, 4096), (4, 4096, 4096), (16, 512, 1024), (3, 300, 8192),
                                   (2, 64, 2048), (5, 33, 100), (1, 16, 16)])
def test_gemv_fp8_shapes_bias(tq, oracle, m, n, k):
    """Weight-only FP8 decode GEMV: y = x . dequant(W)^T + b with f32 x."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    w = normal(78, (n, k), 0.02)
    x = normal(78, (m, k), 1.0, stream=1)
    b = normal(78, (n,), 0.1, stream=2)
    q, s = tq.quantize_per_channel_fp8(dev_tensor(w))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    xd, bd = dev_tensor(x), dev_tensor(b)  # held until the kernel has run
    _abi.call("tq_gemv_fp8", ptr(xd), m, ptr(q), ptr(s), ptr(bd), n, k, ptr(y), stream())
    rq, rs = oracle.quantize_fp8_rowwise(w)
    assert np.array_equal(host(q), rq)
    ref = oracle.linear(x.astype(np.float64), oracle.dequantize_fp8_rowwise(rq, rs).astype(np.float64), b)
    assert_close(host(y), ref, RTOL, ATOL, f"gemv_fp8 {m}x{n}x{k}")


@pytest.mark.parametrize("m", [1, 3, 16, 17, 40])
def test_quantized_linear_fp8_decode_and_weight_only(tq, oracle, m):
    """fp8 mode (the fused GEMV up to 2 tokens, quantize + the skinny GEMM to 16,
    the tiled GEMM above) gives the FP8 W8A8 product; fp8_weight mode gives
    Linear over the dequantized weight with f32 activations."""
    from theano_quantize import QConfig, QuantDType

    n, k = 384, 1024
    w = normal(79, (n, k), 0.02)
    x = normal(79, (m, k), 1.0, stream=1)
    b = normal(79, (n,), 0.1, stream=2)
    rqw, rsw = oracle.quantize_fp8_rowwise(w)
    rqa, rsa = oracle.quantize_fp8_rowwise(x)
    lin = tq.QuantizedLinear.from_tensors(dev_tensor(w), dev_tensor(b), QConfig(QuantDType.FP8, QuantDType.FP8, True,
                                                                                 True))
    assert_close(host(lin(dev_tensor(x))), oracle.linear_fp8(rqa, rsa, rqw, rsw, b), RTOL, ATOL, "fp8 mode")
    wo = tq.QuantizedLinear.from_tensors(dev_tensor(w), dev_tensor(b), QConfig(QuantDType.FP8, QuantDType.UInt8,
                                                                                True, True))
    assert wo.mode == "fp8_weight"
    ref = oracle.linear(x.astype(np.float64), oracle.dequantize_fp8_rowwise(rqw, rsw).astype(np.float64), b)
    assert_close(host(wo(dev_tensor(x))), ref, RTOL, ATOL, "fp8_weight mode")
