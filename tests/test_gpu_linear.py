"""GPU parity: quantized Linear (GEMV, W8A8 GEMM, W4A16 GEMM) and the
quantized FFN vs the oracle's f64 reference (Linear::forward over the
dequantized weight).  Integer accumulators are bit-exact; float outputs are
checked at |got - ref| <= 1e-4 + 1e-3 * |ref|.

At the two heaviest configs every output is compared.  W8A8 at M=2048: all
int32 accumulators equal an f64 GEMM of the integer codes (exact, since every
partial sum is an integer below 2^26 < 2^53, whatever the summation order),
all of y is within tolerance of acc * s_row * s_col in f64 (the product of the
dequantized operands), and the oracle's sequential restatement anchors sampled
rows.  The FFN at M=512: all rows against an f64 composition over the
dequantized weights (SiLU as g * 1/(1+exp(-g)), activation.rs:66-79), with the
oracle's rows as the anchor."""
import numpy as np
import pytest

from conftest import assert_close

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


def bf16_dev(bits):
    import torch

    return dev_tensor(bits.view(np.int16)).view(torch.bfloat16)


def to_bf16_bits(x):
    from theano_quantize.synth import f32_to_bf16_bits

    return f32_to_bf16_bits(x)


# ------------------------------------------------------------------ GEMV
@pytest.fixture(scope="module")
def c2(tq, oracle):
    """Config 2: INT8 per-channel weight [4096, 4096] ~ N(0, 0.02), x [16, 4096] ~ N(0, 1)."""
    w = normal(1, (4096, 4096), 0.02)
    x = normal(1, (16, 4096), 1.0, stream=1)
    q, s = tq.quantize_per_channel_i8(dev_tensor(w))
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert np.array_equal(host(q), rq) and np.array_equal(host(s), rs)
    ref = oracle.linear_w8(x, rq, rs)
    return x, q, s, ref


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 16])
def test_gemv_w8_config2(tq, c2, m):
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream
    import torch

    x, q, s, ref = c2
    y = torch.empty((m, 4096), dtype=torch.float32, device="cuda")
    xd = dev_tensor(x[:m])
    _abi.call("tq_gemv_w8", ptr(xd), m, ptr(q), ptr(s), None, 4096, 4096, ptr(y), stream())
    assert_close(host(y), ref[:m], RTOL, ATOL, f"gemv_w8 M={m}")


# K % 16 != 0 and K > 8192 take the shape-general kernel (e.g. the reference's Linear(3, 2));
# 2-4 tokens with K split over a wave pair: a second half with fewer chunks (K = 3088,
# 3072), rows per pair capped at the LDS partials' 64 (N = 70000 at K = 4096 with 3 tokens
# and K = 8192 with 2: more than 1024 pair runs, so the grid grows past the 256 CUs); runs of
# several row groups per wave, in even and odd numbers, through the two alternating
# register buffers (N = 14336 and 30000 at one token: 7 and 15 rows per wave; N = 9000 at
# two tokens: 3 groups of 2 rows)
@pytest.mark.parametrize("n,k,m", [(1000, 1024, 1), (17, 16, 2), (333, 3088, 3), (64, 8192, 4), (5, 2000, 16),
                                   (2, 3, 4), (50, 100, 3), (64, 9000, 2), (70000, 2048, 3), (4100, 3072, 4),
                                   (515, 8192, 2), (14336, 4096, 1), (30000, 1024, 1), (9000, 1024, 2),
                                   (8192, 2048, 1), (70000, 4096, 3), (70000, 8192, 2)])
def test_gemv_w8_shapes_bias(tq, oracle, n, k, m):
    w = normal(50, (n, k), 0.02)
    x = normal(50, (m, k), 1.0, stream=1)
    b = normal(50, (n,), 0.1, stream=2)
    lin = tq.QuantizedLinear.from_tensors(dev_tensor(w), dev_tensor(b), tq.QConfig.default_int8())
    y = host(lin(dev_tensor(x)))
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert_close(y, oracle.linear_w8(x, rq, rs, b), RTOL, ATOL, f"QuantizedLinear w8 {n}x{k} M={m}")


@pytest.fixture(scope="module")
def c3(tq, oracle):
    """Config 3: INT4 g128 weight [14336, 4096] ~ N(0, 0.02), x bf16 [16, 4096] ~ N(0, 1)."""
    w = normal(2, (14336, 4096), 0.02)
    xb = to_bf16_bits(normal(2, (16, 4096), 1.0, stream=1))
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    rp, rs = oracle.quantize_i4_g128(w)
    assert np.array_equal(host(p), rp) and np.array_equal(host(s).view(np.uint16), rs)
    ref = oracle.linear_w4g128_bf16(xb, rp, rs)
    return xb, p, s, ref


@pytest.mark.parametrize("m", [1, 2, 3, 4, 8, 16])
def test_gemv_w4g128_config3(tq, c3, m):
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream
    import torch

    xb, p, s, ref = c3
    y = torch.empty((m, 14336), dtype=torch.float32, device="cuda")
    xd = bf16_dev(xb[:m])
    _abi.call("tq_gemv_w4g128", ptr(xd), m, ptr(p), ptr(s), None, 14336, 4096, ptr(y), stream())
    assert_close(host(y), ref[:m], RTOL, ATOL, f"gemv_w4g128 M={m}")


def untile(pt, st, n, k, t):
    """Inverse of the row-tiled kernel layout (numpy), for bit-exact checks."""
    tiles = (n + t - 1) // t
    p = pt.reshape(tiles, k // 32, t, 16).transpose(0, 2, 1, 3).reshape(tiles * t, k // 2)
    s = st.reshape(tiles, k // 128, t).transpose(0, 2, 1).reshape(tiles * t, k // 128)
    return p, s


@pytest.mark.parametrize("n,k,t", [(14336, 4096, None), (100, 256, 8), (77, 1024, 64), (4096, 4096, None)])
def test_repack_tiled_is_a_permutation(tq, n, k, t):
    w = normal(57, (n, k), 0.02)
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    pt, st, tr = tq.repack_i4_g128_tiled(p, s, t)
    assert tr % 8 == 0 and 8 <= tr <= 64
    up, us = untile(host(pt), host(st).view(np.uint16), n, k, tr)
    assert np.array_equal(up[:n], host(p)) and np.array_equal(us[:n], host(s).view(np.uint16))
    assert not up[n:].any() and not us[n:].any()  # padding rows are zero


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11, 16])
def test_gemv_w4g128_tiled_config3(tq, c3, m):
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream
    import torch

    xb, p, s, ref = c3
    pt, st, t = tq.repack_i4_g128_tiled(p, s)
    y = torch.empty((m, 14336), dtype=torch.float32, device="cuda")
    xd = bf16_dev(xb[:m])
    _abi.call("tq_gemv_w4g128_tiled", ptr(xd), m, ptr(pt), ptr(st), None, 14336, 4096, t, ptr(y), stream())
    assert_close(host(y), ref[:m], RTOL, ATOL, f"gemv_w4g128_tiled M={m} T={t}")


# Tiles of 16, 32 or 64 rows: 1-4 tokens run the diagonal MFMA kernel (one to
# eight groups per wave, waves past K, tail tiles); 5-16 tokens the MFMA kernel
# with x from L2 (token passes, K <= 8192); other tile heights run the dot2
# kernel.
@pytest.mark.parametrize("n,k,m,t", [(100, 128, 1, 8), (7, 2176, 2, 8), (256, 14336, 1, 16), (48, 16384, 3, 24),
                                     (1000, 4096, 4, 64), (333, 640, 2, 40),
                                     (1000, 4096, 5, 64), (70, 1024, 16, 16), (200, 6144, 7, 32),
                                     (130, 8192, 9, 16), (77, 384, 13, 64), (64, 8192, 3, 64),
                                     (100, 128, 1, 16), (200, 6144, 2, 32), (40, 16384, 2, 32), (333, 4224, 2, 64),
                                     (1000, 4096, 1, 64), (130, 8192, 4, 16), (70, 1152, 3, 16), (100, 2048, 3, 32),
                                     (48, 16384, 3, 16), (4100, 14336, 2, 16), (90, 16384, 1, 64),
                                     (90, 16384, 4, 64), (50, 9000 // 128 * 128, 3, 64)])
def test_gemv_w4g128_tiled_shapes(tq, oracle, n, k, m, t):
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream
    import torch

    w = normal(58, (n, k), 0.02)
    xb = to_bf16_bits(normal(58, (m, k), 1.0, stream=1))
    b = normal(58, (n,), 0.1, stream=2)
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    pt, st, tr = tq.repack_i4_g128_tiled(p, s, t)
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    bd, xd = dev_tensor(b), bf16_dev(xb)
    _abi.call("tq_gemv_w4g128_tiled", ptr(xd), m, ptr(pt), ptr(st), ptr(bd), n, k, tr, ptr(y), stream())
    rp, rs = oracle.quantize_i4_g128(w)
    assert_close(host(y), oracle.linear_w4g128_bf16(xb, rp, rs, b), RTOL, ATOL, f"tiled {n}x{k} M={m} T={t}")


# QuantizedLinear "w4" up to M = 32 runs the tiled GEMV in passes of 16 tokens
# (17 and 32 below; 40 and 64 take the prefill GEMM)
@pytest.mark.parametrize("n,k,m", [(100, 128, 1), (7, 2176, 2), (256, 14336, 1), (48, 16384, 3), (9, 4096, 16),
                                   (33, 16512, 2), (100, 1024, 17), (256, 2048, 32), (9, 4096, 40),
                                   (300, 2048, 64)])
def test_gemv_w4g128_shapes_bias(tq, oracle, n, k, m):
    w = normal(51, (n, k), 0.02)
    xb = to_bf16_bits(normal(51, (m, k), 1.0, stream=1))
    b = normal(51, (n,), 0.1, stream=2)
    lin = tq.QuantizedLinear.from_tensors(dev_tensor(w), dev_tensor(b), tq.QConfig.default_int4())
    y = host(lin(bf16_dev(xb)))
    rp, rs = oracle.quantize_i4_g128(w)
    assert_close(y, oracle.linear_w4g128_bf16(xb, rp, rs, b), RTOL, ATOL, f"QuantizedLinear w4 {n}x{k} M={m}")


# ------------------------------------------------------------------ W8A8
def checksums_ok(acc, qa, qw, seed=0):
    a = qa.astype(np.int64)
    w = qw.astype(np.int64)
    acc = acc.astype(np.int64)
    rows = np.array_equal(acc.sum(axis=1), a @ w.sum(axis=0))
    cols = np.array_equal(acc.sum(axis=0), a.sum(axis=0) @ w.T)
    r = np.random.default_rng(seed).integers(-3, 4, acc.shape[1]).astype(np.int64)
    proj = np.array_equal(acc @ r, a @ (w.T @ r))
    return rows and cols and proj


def run_w8a8(tq, x, w, bias=None, with_acc=True):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    m, k = x.shape
    n = w.shape[0]
    qa, sa = tq.quantize_per_channel_i8(dev_tensor(x))
    qw, sw = tq.quantize_per_channel_i8(dev_tensor(w))
    acc = torch.empty((m, n), dtype=torch.int32, device="cuda") if with_acc else None
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    bd = None if bias is None else dev_tensor(bias)
    _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), ptr(bd), m, n, k, ptr(acc), ptr(y), stream())
    return host(qa), host(sa), host(qw), host(sw), (host(acc) if with_acc else None), host(y)


def test_w8a8_config4_full(tq, oracle):
    x = normal(3, (2048, 4096), 1.0)
    w = normal(3, (4096, 4096), 0.02, stream=1)
    qa, sa, qw, sw, acc, y = run_w8a8(tq, x, w)
    rqa, rsa = oracle.quantize_i8_rowwise(x)
    rqw, rsw = oracle.quantize_i8_rowwise(w)
    assert np.array_equal(qa, rqa) and np.array_equal(sa, rsa)
    assert np.array_equal(qw, rqw) and np.array_equal(sw, rsw)
    assert checksums_ok(acc, qa, qw)
    acc_ref = qa.astype(np.float64) @ qw.astype(np.float64).T
    assert np.abs(acc_ref).max() < 2.0 ** 26
    bad = acc.astype(np.float64) != acc_ref
    assert not bad.any(), f"{int(bad.sum())} of {acc.size} int32 accumulators differ, first at {np.argwhere(bad)[0]}"
    y_ref = acc_ref * sa.astype(np.float64)[:, None] * sw.astype(np.float64)[None, :]
    assert_close(y, y_ref, RTOL, ATOL, "w8a8 y (all rows)")
    rows = np.array([0, 1, 127, 128, 1000, 2047])
    assert np.array_equal(acc[rows], oracle.gemm_w8a8_acc(qa[rows], qw))
    assert_close(y[rows], oracle.linear_w8a8(qa[rows], sa[rows], qw, sw), RTOL, ATOL, "w8a8 y vs oracle")


# M <= 16 with K % 64 == 0 (K <= 8192) takes the skinny kernel (one to eight
# chunks per wave, waves past K, one-block grids); K % 128 == 0 the LDS-DMA kernel
# (1, 2, 3 and more stages; M, N tails; tile groups with and without the XCD
# remap), other K the general kernel.
@pytest.mark.parametrize("m,n,k", [(1, 16, 16), (130, 48, 208), (64, 160, 80),
                                   (7, 272, 1024), (257, 128, 4096), (300, 512, 128),
                                   (129, 4096, 256), (100, 272, 384), (384, 2048, 256),
                                   (1, 256, 640), (1031, 528, 512),
                                   (5, 8, 256), (33, 50, 100), (17, 16, 1000),
                                   (16, 4096, 4096), (3, 64, 8192), (16, 16, 64), (9, 1024, 192),
                                   (2, 48, 4096), (16, 32, 8256)])
def test_w8a8_shapes_bias(tq, oracle, m, n, k):
    x = normal(52, (m, k), 1.0)
    w = normal(52, (n, k), 0.02, stream=1)
    b = normal(52, (n,), 0.1, stream=2)
    qa, sa, qw, sw, acc, y = run_w8a8(tq, x, w, b)
    assert np.array_equal(acc, oracle.gemm_w8a8_acc(qa, qw))
    assert_close(y, oracle.linear_w8a8(qa, sa, qw, sw, b), RTOL, ATOL, f"w8a8 {m}x{n}x{k}")
    _, _, _, _, _, y2 = run_w8a8(tq, x, w, b, with_acc=False)
    assert np.array_equal(y, y2)


def test_w8a8_extreme_codes(tq, oracle):
    # every code -128/127 paths: rows of constant sign reach |acc| = K*127*128
    x = np.where(normal(53, (32, 4096), 1.0) > 0, 1.0, -1.0).astype(np.float32)
    w = np.where(normal(53, (64, 4096), 1.0, stream=1) > 0, 1.0, -1.0).astype(np.float32)
    x[0] = 1.0
    w[0] = 1.0
    qa, sa, qw, sw, acc, y = run_w8a8(tq, x, w)
    assert np.array_equal(acc, oracle.gemm_w8a8_acc(qa, qw))
    assert acc[0, 0] == 4096 * 127 * 127


# M = 1, 2: the fused GEMV; 3, 16: quantize + the skinny GEMM; 100: the tiled GEMM
@pytest.mark.parametrize("m", [1, 2, 3, 16, 100])
def test_quantized_linear_w8a8_module(tq, oracle, m):
    from theano_quantize import QConfig, QuantDType

    w = normal(54, (256, 512), 0.02)
    x = normal(54, (m, 512), 1.0, stream=1)
    cfg = QConfig(QuantDType.Int8, QuantDType.Int8, True, True)
    lin = tq.QuantizedLinear.from_tensors(dev_tensor(w), None, cfg)
    y = host(lin(dev_tensor(x)))
    rqa, rsa = oracle.quantize_i8_rowwise(x)
    rqw, rsw = oracle.quantize_i8_rowwise(w)
    assert_close(y, oracle.linear_w8a8(rqa, rsa, rqw, rsw), RTOL, ATOL, "QuantizedLinear w8a8")
    assert lin.num_parameters() == 256 * 512


def test_misaligned_inputs_take_the_general_kernels(tq, oracle):
    """Device views that start off a 16-byte boundary still give the oracle's result."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    m, n, k = 3, 40, 256
    w = normal(57, (n, k), 0.02)
    x = normal(57, (m, k), 1.0, stream=1)
    q, s = tq.quantize_per_channel_i8(dev_tensor(w))
    big = torch.zeros(m * k + 1, dtype=torch.float32, device="cuda")
    xv = big[1:].view(m, k)
    xv.copy_(dev_tensor(x))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _abi.call("tq_gemv_w8", ptr(xv), m, ptr(q), ptr(s), None, n, k, ptr(y), stream())
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert_close(host(y), oracle.linear_w8(x, rq, rs), RTOL, ATOL, "gemv_w8 misaligned x")
    xb = to_bf16_bits(x)
    p4, s4 = tq.quantize_i4_g128(dev_tensor(w))
    bigb = torch.zeros(m * k + 1, dtype=torch.int16, device="cuda")
    xbv = bigb[1:].view(m, k)
    xbv.copy_(dev_tensor(xb.view(np.int16)))
    _abi.call("tq_gemv_w4g128", ptr(xbv), m, ptr(p4), ptr(s4), None, n, k, ptr(y), stream())
    rp, rs4 = oracle.quantize_i4_g128(w)
    assert_close(host(y), oracle.linear_w4g128_bf16(xb, rp, rs4), RTOL, ATOL, "gemv_w4 misaligned x")


# ----------------------------------------------------------------- W4A16
# (17, 256, 512), (300, 512, 768), (64, 1024, 4096), (129, 768, 2048) and
# (64, 384, 1024) run the pipelined kernels on 64 x 128 tiles (K split in two
# where the grid is small; N = 384 has no 256-column tiling); (512, 16384, 256)
# on 128 x 256 tiles (as many rounds of work per CU either way: the wide tiles
# win the tie); the rest the 16x16x32 / shape-general kernels.  The layer has
# no tiled copy, so that every M takes the prefill GEMM.
@pytest.mark.parametrize("m,n,k", [(17, 256, 512), (130, 64, 4096), (300, 128, 1024), (33, 16, 128),
                                   (40, 200, 1024), (20, 7, 256), (300, 512, 768), (64, 1024, 4096),
                                   (129, 768, 2048), (64, 384, 1024), (512, 16384, 256)])
def test_gemm_w4g128_bf16_shapes(tq, oracle, m, n, k):
    w = normal(55, (n, k), 0.02)
    xb = to_bf16_bits(normal(55, (m, k), 1.0, stream=1))
    b = normal(55, (n,), 0.1, stream=2)
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    lin = tq.QuantizedLinear("w4", k, n, p, s, dev_tensor(b), tiled=False)
    assert lin.tiled is None
    y = host(lin(bf16_dev(xb)))
    rp, rs = oracle.quantize_i4_g128(w)
    assert_close(y, oracle.linear_w4g128_bf16(xb, rp, rs, b), RTOL, ATOL, f"w4a16 {m}x{n}x{k}")


# ------------------------------------------------------------------- MLP
def _prefill_only(tq, mlp):
    """The same weights without the decode copies: every M runs the prefill kernels."""
    return tq.QuantizedMLP(mlp.d, mlp.f, mlp.gate, mlp.up, mlp.down, tiled=False)


# Prefill kernels: (5, 256, 384) and (1, 128, 128) have an odd number of groups:
# shape-general path; the others take the pipelined kernels (row tails at 64 / 128).
@pytest.mark.parametrize("m,d,f", [(5, 256, 384), (1, 128, 128), (70, 512, 1024), (1, 256, 512),
                                   (129, 768, 1536), (300, 1024, 2048), (64, 256, 256), (200, 512, 768)])
def test_mlp_small(tq, oracle, m, d, f):
    wg = normal(56, (f, d), 0.02)
    wu = normal(56, (f, d), 0.02, stream=1)
    wd = normal(56, (d, f), 0.02, stream=2)
    xb = to_bf16_bits(normal(56, (m, d), 1.0, stream=3))
    mlp = _prefill_only(tq, tq.QuantizedMLP.from_tensors(dev_tensor(wg), dev_tensor(wu), dev_tensor(wd)))
    y = host(mlp(bf16_dev(xb)))
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    assert_close(y, oracle.mlp_w4g128(xb, *args), RTOL, ATOL, f"mlp {m}x{d}x{f}")


def mlp_f64(xb, pg, sg, pu, su, pd, sd, oracle):
    """The FFN in f64 over the dequantized weights (exact in f32: q * s), as
    numpy matmuls: h = g * 1/(1+exp(-g)) * u, y = h Wd^T."""
    x = (xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    g = x @ oracle.dequantize_i4_g128(pg, sg).astype(np.float64).T
    u = x @ oracle.dequantize_i4_g128(pu, su).astype(np.float64).T
    h = g * (1.0 / (1.0 + np.exp(-g))) * u
    del g, u
    return h @ oracle.dequantize_i4_g128(pd, sd).astype(np.float64).T


def test_mlp_config5_all_rows(tq, oracle):
    d, f, m = 4096, 14336, 512
    wg = normal(4, (f, d), 0.02)
    wu = normal(4, (f, d), 0.02, stream=1)
    wd = normal(4, (d, f), 0.02, stream=2)
    xb = to_bf16_bits(normal(4, (m, d), 1.0, stream=3))
    mlp = tq.QuantizedMLP.from_tensors(dev_tensor(wg), dev_tensor(wu), dev_tensor(wd))
    y = host(mlp(bf16_dev(xb)))
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    # one row in each 128-row M tile of the prefill kernels, plus the last row
    rows = np.array([0, 129, 300, 400, 511])
    ref_rows = oracle.mlp_w4g128(xb[rows], *args)
    assert_close(y[rows], ref_rows, RTOL, ATOL, "mlp config 5 vs oracle")
    ref = mlp_f64(xb, *args, oracle)
    # the f64 composition itself agrees with the oracle's sequential restatement
    assert_close(ref[rows], ref_rows, 1e-9, 1e-9, "f64 composition vs oracle")
    assert_close(y, ref, RTOL, ATOL, "mlp config 5 (all rows)")


@pytest.mark.parametrize("m", [64, 200])
def test_mlp_mid_m_config5_weights(tq, oracle, m):
    """Mid-size M on the prefill kernels at the config-5 weights: M = 64 runs
    gate/up on 64-row tiles and down on 64 x 64 tiles; M = 200 keeps gate/up on
    128-row tiles (a tie in rounds x work) and runs down on 64 x 64 tiles.  All
    rows against the f64 composition, sampled rows against the oracle."""
    d, f = 4096, 14336
    wg = normal(4, (f, d), 0.02)
    wu = normal(4, (f, d), 0.02, stream=1)
    wd = normal(4, (d, f), 0.02, stream=2)
    xb = to_bf16_bits(normal(4, (m, d), 1.0, stream=4))
    mlp = _prefill_only(tq, tq.QuantizedMLP.from_tensors(dev_tensor(wg), dev_tensor(wu), dev_tensor(wd)))
    y = host(mlp(bf16_dev(xb)))
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    rows = np.array([0, 63, m - 1])
    assert_close(y[rows], oracle.mlp_w4g128(xb[rows], *args), RTOL, ATOL, f"mlp M={m} vs oracle")
    assert_close(y, mlp_f64(xb, *args, oracle), RTOL, ATOL, f"mlp M={m} (all rows)")


def _mlp_case(tq, m, d, f, seed=57):
    wg = normal(seed, (f, d), 0.02)
    wu = normal(seed, (f, d), 0.02, stream=1)
    wd = normal(seed, (d, f), 0.02, stream=2)
    xb = to_bf16_bits(normal(seed, (m, d), 1.0, stream=3))
    mlp = tq.QuantizedMLP.from_tensors(dev_tensor(wg), dev_tensor(wu), dev_tensor(wd))
    return mlp, xb


# Decode path (M <= 8, and M <= 32 where D <= 4096, in passes of 16 tokens): gate
# and up interleaved in 64-row tiles with SiLU * up in the epilogue (4 tokens per
# launch up to M = 4; 5-16 tokens in one launch of the 32x32 kernel where D <=
# 4096, else 4 per launch), down on h as bf16 hi + lo rows in 32-row tiles, one
# launch per four tokens (eight at M >= 5) with K split over two blocks per tile
# (including F = 128 where the second block has no groups); one to eight groups
# per wave, F not a multiple of 64, the Llama shape.  At 5-16 tokens the down
# launch stages h through LDS by runs of 1, 2 or 4 groups per wave (the last in
# two phases, F = 13056 leaving a phase half live); at 9-16 tokens one launch
# takes all 2m rows of h through per-group LDS strips (1, 2, 3 and 4 groups per
# wave: F = 640, 6144, 8320, 14336).  Gate/up tiles past the CU count run two per
# block (D = 2560-4096 with F = 8320-16384).
@pytest.mark.parametrize("m,d,f", [(1, 128, 128), (2, 256, 384), (3, 512, 1024), (4, 1024, 640), (5, 256, 512),
                                   (7, 384, 1152), (8, 2048, 256), (1, 4096, 14336), (2, 14336, 4096),
                                   (6, 16384, 128), (3, 4096, 14336), (4, 4096, 14336), (4, 256, 128),
                                   (3, 640, 16384), (6, 4096, 14336), (8, 4096, 14336), (2, 4096, 14336),
                                   (9, 256, 512), (12, 4096, 14336), (16, 1024, 640), (16, 4096, 14336),
                                   (13, 128, 384), (7, 8192, 1024), (17, 4096, 14336), (28, 512, 1536),
                                   (25, 256, 384), (9, 512, 6144), (5, 1024, 8192), (10, 1024, 13056),
                                   (7, 3072, 9216), (11, 2560, 8320), (16, 4096, 16384)])
def test_mlp_decode_path(tq, oracle, m, d, f):
    wg = normal(60, (f, d), 0.02)
    wu = normal(60, (f, d), 0.02, stream=1)
    wd = normal(60, (d, f), 0.02, stream=2)
    xb = to_bf16_bits(normal(60, (m, d), 1.0, stream=3))
    mlp = tq.QuantizedMLP.from_tensors(dev_tensor(wg), dev_tensor(wu), dev_tensor(wd))
    assert mlp._decode_path(m)
    assert mlp._decode_path(28) == (d <= 4096) and not mlp._decode_path(29)
    y = host(mlp(bf16_dev(xb)))
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    assert_close(y, oracle.mlp_w4g128(xb, *args), RTOL, ATOL, f"mlp decode {m}x{d}x{f}")


# The C ABI takes down copies of 16, 32 or 64 rows per tile.  16-row tiles run
# the down projection per token pair (M = 1-2, 5-8) or per four tokens with K
# split in two (M = 3-4); 64-row tiles always per token pair.
@pytest.mark.parametrize("tile_rows", [16, 64])
@pytest.mark.parametrize("m,d,f", [(1, 512, 1536), (2, 256, 384), (3, 512, 1024), (4, 1024, 640), (5, 256, 512),
                                   (8, 384, 1152), (4, 4096, 14336), (2, 4096, 14336), (3, 640, 16384)])
def test_mlp_decode_down_tile_heights(tq, oracle, tile_rows, m, d, f):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    print(f"decode FFN, {tile_rows}-row down tiles: M={m} D={d} F={f}", flush=True)
    mlp, xb = _mlp_case(tq, m, d, f, seed=63)
    gu_t, gu_st, _, _, _ = mlp.decode
    dn_t, dn_st, t = tq.repack_i4_g128_tiled(mlp.down[0], mlp.down[1], tile_rows)
    assert t == tile_rows
    nb = int(_abi.lib().tq_mlp_w4g128_decode_workspace_bytes(m, d, f))
    ws = torch.empty((nb,), dtype=torch.uint8, device="cuda")
    x = bf16_dev(xb)
    y = torch.full((m, d), float("nan"), dtype=torch.float32, device="cuda")
    _abi.call("tq_mlp_w4g128_decode", ptr(x), m, d, f, ptr(gu_t), ptr(gu_st), ptr(dn_t), ptr(dn_st), tile_rows,
              ptr(ws), nb, ptr(y), stream())
    args = [a for w in (mlp.gate, mlp.up, mlp.down) for a in (host(w[0]), host(w[1]).view(np.uint16))]
    assert_close(host(y), oracle.mlp_w4g128(xb, *args), RTOL, ATOL, f"mlp decode {tile_rows}-row down, {m}x{d}x{f}")


# The decode FFN takes x rows 8-byte aligned (the gate/up kernels load x in 8-byte
# pieces): the same result as from a 16-byte aligned copy, at 5-16 tokens (one
# and two gate/up tiles per block) and with the one-launch down projection.
@pytest.mark.parametrize("m,d,f", [(6, 4096, 14336), (12, 4096, 14336), (16, 1024, 640), (9, 512, 6144)])
def test_mlp_decode_x_8_byte_aligned(tq, oracle, m, d, f):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    print(f"decode FFN, x 8-byte aligned: M={m} D={d} F={f}", flush=True)
    mlp, xb = _mlp_case(tq, m, d, f, seed=64)
    gu_t, gu_st, dn_t, dn_st, t = mlp.decode
    nb = int(_abi.lib().tq_mlp_w4g128_decode_workspace_bytes(m, d, f))
    ws = torch.empty((nb,), dtype=torch.uint8, device="cuda")
    buf = torch.zeros(m * d + 4, dtype=torch.bfloat16, device="cuda")
    x = buf[4:].view(m, d)
    x.copy_(bf16_dev(xb))
    assert x.data_ptr() % 16 == 8
    args = [a for w in (mlp.gate, mlp.up, mlp.down) for a in (host(w[0]), host(w[1]).view(np.uint16))]
    ref = oracle.mlp_w4g128(xb, *args)
    for xin in (x, bf16_dev(xb)):
        y = torch.full((m, d), float("nan"), dtype=torch.float32, device="cuda")
        _abi.call("tq_mlp_w4g128_decode", ptr(xin), m, d, f, ptr(gu_t), ptr(gu_st), ptr(dn_t), ptr(dn_st), t,
                  ptr(ws), nb, ptr(y), stream())
        assert_close(host(y), ref, RTOL, ATOL, f"mlp decode {m}x{d}x{f}, x at {xin.data_ptr() % 16} mod 16")


def test_mlp_decode_and_prefill_agree_and_reuse_workspace(tq, oracle):
    """Both paths meet the tolerance on the same weights; one decode workspace
    serves calls of decreasing M; a short one is rejected."""
    import torch
    from theano_quantize import InvalidArgument

    d, f = 512, 1536
    mlp, xb = _mlp_case(tq, 8, d, f, seed=61)
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    ws = torch.empty((mlp.workspace_bytes(8),), dtype=torch.uint8, device="cuda")
    pre = _prefill_only(tq, mlp)
    for m in (8, 5, 4, 3, 2, 1):
        ref = oracle.mlp_w4g128(xb[:m], *args)
        assert_close(host(mlp.forward(bf16_dev(xb[:m]), ws)), ref, RTOL, ATOL, f"decode M={m}")
        assert_close(host(pre.forward(bf16_dev(xb[:m]))), ref, RTOL, ATOL, f"prefill M={m}")
    with pytest.raises(InvalidArgument):
        mlp.forward(bf16_dev(xb), ws[:mlp.workspace_bytes(8) - 256])


def test_repack_gate_up_is_a_permutation(tq):
    """Tile t of the gate/up copy: gate rows 32t..32t+31, then the same up rows, in
    the row-tiled layout with 64-row tiles; rows past F are zero."""
    f, d = 96, 384
    p_g, s_g = tq.quantize_i4_g128(dev_tensor(normal(62, (f, d), 0.02)))
    p_u, s_u = tq.quantize_i4_g128(dev_tensor(normal(62, (f, d), 0.02, stream=1)))
    pt, st = tq.repack_i4_g128_gate_up_tiled((p_g, s_g), (p_u, s_u))
    tiles = (f + 31) // 32
    up, us = untile(host(pt), host(st).view(np.uint16), tiles * 64, d, 64)
    pg, pu = np.zeros((tiles * 32, d // 2), np.uint8), np.zeros((tiles * 32, d // 2), np.uint8)
    sg, su = np.zeros((tiles * 32, d // 128), np.uint16), np.zeros((tiles * 32, d // 128), np.uint16)
    pg[:f], pu[:f] = host(p_g), host(p_u)
    sg[:f], su[:f] = host(s_g).view(np.uint16), host(s_u).view(np.uint16)
    for t in range(tiles):
        assert np.array_equal(up[64 * t:64 * t + 32], pg[32 * t:32 * t + 32])
        assert np.array_equal(up[64 * t + 32:64 * t + 64], pu[32 * t:32 * t + 32])
        assert np.array_equal(us[64 * t:64 * t + 32], sg[32 * t:32 * t + 32])
        assert np.array_equal(us[64 * t + 32:64 * t + 64], su[32 * t:32 * t + 32])


def test_mlp_paths_agree(tq, oracle):
    """A workspace that is 16- but not 256-byte aligned selects the shape-general
    kernels; both paths meet the tolerance against the oracle."""
    import torch

    m, d, f = 96, 512, 1024
    mlp, xb = _mlp_case(tq, m, d, f)
    need = mlp.workspace_bytes(m)
    raw = torch.empty((need + 256,), dtype=torch.uint8, device="cuda")
    assert raw.data_ptr() % 256 == 0
    y_fast = host(mlp.forward(bf16_dev(xb), raw[:need]))
    y_gen = host(mlp.forward(bf16_dev(xb), raw[16:16 + need]))
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    ref = oracle.mlp_w4g128(xb, *args)
    assert_close(y_fast, ref, RTOL, ATOL, "mlp pipelined")
    assert_close(y_gen, ref, RTOL, ATOL, "mlp shape-general")


def test_mlp_workspace_reuse_and_size_check(tq, oracle):
    """One workspace serves calls of decreasing M (stale intermediates of a larger
    call must not leak into a smaller one); a short workspace is rejected."""
    import torch
    from theano_quantize import InvalidArgument

    d, f = 256, 512
    mlp, xb = _mlp_case(tq, 300, d, f, seed=58)
    mlp = _prefill_only(tq, mlp)
    ws = torch.empty((mlp.workspace_bytes(300),), dtype=torch.uint8, device="cuda")
    args = [a for t in (mlp.gate, mlp.up, mlp.down) for a in (host(t[0]), host(t[1]).view(np.uint16))]
    for m in (300, 130, 7):
        y = host(mlp.forward(bf16_dev(xb[:m]), ws))
        assert_close(y, oracle.mlp_w4g128(xb[:m], *args), RTOL, ATOL, f"mlp reuse M={m}")
    short = torch.empty((mlp.workspace_bytes(300) - 256,), dtype=torch.uint8, device="cuda")
    with pytest.raises(InvalidArgument):
        mlp.forward(bf16_dev(xb), short)


def test_gemm_w4g128_bf16_entry_points_agree(tq, oracle):
    """The workspace entry point (pipelined kernels) and the workspace-free one
    (16x16x32 kernel) both meet the tolerance; a short workspace is rejected."""
    import torch
    from theano_quantize import InvalidArgument, _abi
    from theano_quantize._tensor import ptr, stream

    m, n, k = 200, 512, 2048
    w = normal(59, (n, k), 0.02)
    b = normal(59, (n,), 0.1, stream=2)
    xb = to_bf16_bits(normal(59, (m, k), 1.0, stream=1))
    q, s = tq.quantize_i4_g128(dev_tensor(w))
    x, bias = bf16_dev(xb), dev_tensor(b)
    y1 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    y2 = torch.empty_like(y1)
    nb = int(_abi.lib().tq_gemm_w4g128_bf16_workspace_bytes(m, k))
    ws = torch.empty((nb,), dtype=torch.uint8, device="cuda")
    _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), m, ptr(q), ptr(s), ptr(bias), n, k, ptr(ws), nb, ptr(y1), stream())
    _abi.call("tq_gemm_w4g128_bf16", ptr(x), m, ptr(q), ptr(s), ptr(bias), n, k, ptr(y2), stream())
    rp, rs = oracle.quantize_i4_g128(w)
    ref = oracle.linear_w4g128_bf16(xb, rp, rs, b)
    assert_close(host(y1), ref, RTOL, ATOL, "w4a16 pipelined")
    assert_close(host(y2), ref, RTOL, ATOL, "w4a16 16x16x32")
    with pytest.raises(InvalidArgument):
        _abi.call("tq_gemm_w4g128_bf16_ws", ptr(x), m, ptr(q), ptr(s), ptr(bias), n, k, ptr(ws), nb - 256,
                  ptr(y1), stream())


# ------------------------------------------ decode W8A8 / FP8, fused activations
@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (3, 512, 1024), (16, 272, 8192), (5, 33, 48), (2, 4096, 128),
                                   (1, 14336, 4096), (1, 30000, 1024)])
def test_gemv_w8a8_fused_equals_quantize_plus_gemm(tq, oracle, m, n, k):
    """One launch (activation codes computed in the GEMV) gives the two-step
    path's y bit for bit: same codes, exact int32 sums, same epilogue."""
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    x = normal(61, (m, k), 1.0)
    x[0, :5] = [0.0, -0.0, np.nan, 3e4, -3e4]
    w = normal(61, (n, k), 0.02, stream=1)
    b = normal(61, (n,), 0.1, stream=2)
    xd, bd = dev_tensor(x), dev_tensor(b)
    qw, sw = tq.quantize_per_channel_i8(dev_tensor(w))
    y1 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _abi.call("tq_gemv_w8a8", ptr(xd), m, ptr(qw), ptr(sw), ptr(bd), n, k, ptr(y1), stream())
    qa, sa = tq.quantize_per_channel_i8(xd)
    y2 = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _abi.call("tq_gemm_w8a8", ptr(qa), ptr(sa), ptr(qw), ptr(sw), ptr(bd), m, n, k, None, ptr(y2), stream())
    assert np.array_equal(host(y1), host(y2))
    rqa, rsa = oracle.quantize_i8_rowwise(x)
    rqw, rsw = oracle.quantize_i8_rowwise(w)
    assert_close(host(y1), oracle.linear_w8a8(rqa, rsa, rqw, rsw, b), RTOL, ATOL, "fused w8a8 vs oracle")


@pytest.mark.parametrize("m,n,k", [(1, 4096, 4096), (4, 512, 1024), (16, 272, 8192), (3, 40, 64), (1, 14336, 2048)])
def test_gemv_fp8a8_fused_vs_oracle(tq, oracle, m, n, k):
    import torch
    from theano_quantize import _abi
    from theano_quantize._tensor import ptr, stream

    x = normal(62, (m, k), 1.0)
    w = normal(62, (n, k), 0.02, stream=1)
    b = normal(62, (n,), 0.1, stream=2)
    xd, bd = dev_tensor(x), dev_tensor(b)
    qw, sw = tq.quantize_per_channel_fp8(dev_tensor(w))
    y = torch.empty((m, n), dtype=torch.float32, device="cuda")
    _abi.call("tq_gemv_fp8a8", ptr(xd), m, ptr(qw), ptr(sw), ptr(bd), n, k, ptr(y), stream())
    rqa, rsa = oracle.quantize_fp8_rowwise(x)
    rqw, rsw = oracle.quantize_fp8_rowwise(w)
    assert_close(host(y), oracle.linear_fp8(rqa, rsa, rqw, rsw, b), RTOL, ATOL, "fused fp8 vs oracle")
