"""GPU parity: quantize / dequantize kernels vs the C oracle, bit-exact.

Runs the HIP path through the C ABI (theano_quantize -> libtq.so) on seeded
inputs and compares every code, packed byte and scale with the oracle.  Full
BASELINE sizes are used where the oracle finishes in seconds (config 1:
W [4096, 4096]; config 3 weights: [14336, 4096])."""
import math

import numpy as np
import pytest

from conftest import ieee_equal

pytestmark = pytest.mark.gpu


def dev_tensor(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    import torch

    torch.cuda.synchronize()
    return t.cpu().numpy()


def weights(seed, shape, std=0.02, stream=0):
    from theano_quantize.synth import normal_f32

    return normal_f32(seed, shape, std, stream)


def tie_row(k):
    """A row whose absmax is 127/128, so s = 2^-7 exactly and x = (j + 1/2) s are ties."""
    j = np.arange(k) % 254 - 127
    x = ((j + 0.5) * 2.0 ** -7).astype(np.float32)
    x[0] = np.float32(127.0 / 128.0)
    return np.clip(x, -127.0 / 128.0, 127.0 / 128.0).astype(np.float32)


# -------------------------------------------------------- per-row INT8
def test_quantize_i8_rowwise_config1_full(tq, oracle):
    w = weights(0, (4096, 4096))
    q, s, d = tq.fake_quantize_per_channel_i8(dev_tensor(w))
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert np.array_equal(host(s), rs)
    assert np.array_equal(host(q), rq)
    assert ieee_equal(host(d), oracle.dequantize_i8_rowwise(rq, rs))
    q2, s2 = tq.quantize_per_channel_i8(dev_tensor(w))
    assert np.array_equal(host(q2), rq) and np.array_equal(host(s2), rs)
    assert ieee_equal(host(tq.dequantize_per_channel_i8(q2, s2)), oracle.dequantize_i8_rowwise(rq, rs))


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (7, 100), (5, 4097), (2, 20000), (33, 1024),
                                   (9, 4), (4, 16384), (3, 16388)])
def test_quantize_i8_rowwise_ragged(tq, oracle, shape):
    w = weights(20, shape, std=1.0)
    q, s, d = tq.fake_quantize_per_channel_i8(dev_tensor(w))
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert np.array_equal(host(s), rs) and np.array_equal(host(q), rq)
    assert ieee_equal(host(d), oracle.dequantize_i8_rowwise(rq, rs))


# K = 2048 and 4096 run the 4-wave-per-row kernel with the dequantized copy
@pytest.mark.parametrize("k", [512, 2048, 4096])
def test_quantize_i8_rowwise_special_rows(tq, oracle, k):
    rows = [np.zeros(k, np.float32), tie_row(k), -tie_row(k), weights(21, (k,), 1.0)]
    nanrow = weights(22, (k,), 1.0)
    nanrow[::7] = np.nan
    infrow = weights(23, (k,), 1.0)
    infrow[3] = np.inf
    allnan = np.full(k, np.nan, np.float32)
    tiny = (weights(24, (k,), 1.0) * 1e-38).astype(np.float32)  # subnormal inputs
    w = np.stack(rows + [nanrow, infrow, allnan, tiny])
    for wv in (w, w[:, :500]):  # vector and generic kernels
        wv = np.ascontiguousarray(wv)
        q, s, d = tq.fake_quantize_per_channel_i8(dev_tensor(wv))
        rq, rs = oracle.quantize_i8_rowwise(wv)
        assert ieee_equal(host(s), rs)
        assert np.array_equal(host(q), rq)
        assert ieee_equal(host(d), oracle.dequantize_i8_rowwise(rq, rs))
    assert host(s)[0] == np.float32(1e-10)
    rq, rs = oracle.quantize_i8_rowwise(np.ascontiguousarray(w[1:2]))
    assert rs[0] == np.float32(2.0 ** -7)
    j = np.arange(k) % 254 - 127  # x = (j + 1/2) s: ties go away from zero
    expect = np.where(j >= 0, j + 1, j)
    expect[0] = 127
    assert np.array_equal(rq[0].astype(np.int64), expect)


# Codes only with 1025-4096 elements per row and at most 8 rows per CU runs a wave
# per row (K a multiple of 16 but not of 256: masked lanes) or a row per 4-wave
# block (K = 2048, 4096), with ties, NaN, inf, all-NaN and subnormal rows, up to
# 2048 rows.
@pytest.mark.parametrize("rows,k", [(9, 1040), (9, 2064), (9, 4096), (2048, 1296), (1999, 2048)])
def test_quantize_rowwise_codes_only_wave_rows(tq, oracle, rows, k):
    base = [np.zeros(k, np.float32), tie_row(k), -tie_row(k)]
    nanrow = weights(26, (k,), 1.0)
    nanrow[::7] = np.nan
    infrow = weights(27, (k,), 1.0)
    infrow[k - 1] = -np.inf
    allnan = np.full(k, np.nan, np.float32)
    tiny = (weights(28, (k,), 1.0) * 1e-38).astype(np.float32)
    special = np.stack(base + [nanrow, infrow, allnan, tiny])
    w = np.concatenate([special, weights(29, (rows - len(special) if rows > len(special) else 2, k), 1.0)])
    q, s = tq.quantize_per_channel_i8(dev_tensor(w))
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert ieee_equal(host(s), rs) and np.array_equal(host(q), rq)
    q8, s8 = tq.quantize_per_channel_fp8(dev_tensor(w))
    rq8, rs8 = oracle.quantize_fp8_rowwise(w)
    assert ieee_equal(host(s8), rs8) and np.array_equal(host(q8), rq8)


def test_unaligned_and_offset_views(tq, oracle):
    import torch

    w = weights(25, (6, 260), std=1.0)
    buf = torch.empty(6 * 260 + 1, dtype=torch.float32, device="cuda")
    buf[1:] = dev_tensor(w.ravel())
    view = buf[1:].view(6, 260)  # 4-byte aligned, not 16-byte aligned
    q, s = tq.quantize_per_channel_i8(view)
    rq, rs = oracle.quantize_i8_rowwise(w)
    assert np.array_equal(host(q), rq) and np.array_equal(host(s), rs)


# --------------------------------------------------------- INT4 g128
def test_quantize_i4_g128_config3_weights(tq, oracle):
    w = weights(2, (14336, 4096))
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    rp, rs = oracle.quantize_i4_g128(w)
    assert np.array_equal(host(s).view(np.uint16), rs)
    assert np.array_equal(host(p), rp)
    sub = slice(0, 512)
    assert ieee_equal(host(tq.dequantize_i4_g128(p[sub], s[sub])), oracle.dequantize_i4_g128(rp[sub], rs[sub]))


def test_quantize_i4_g128_special_groups(tq, oracle):
    g = 128
    groups = [np.zeros(g, np.float32),                       # floor scale 2^-24
              (weights(30, (g,), 1.0) * 1e-6).astype(np.float32),   # subnormal f16 scale
              (weights(31, (g,), 1.0) * 1e-9).astype(np.float32),   # scale rounds to 0 -> floor
              (weights(32, (g,), 1.0) * 1e6).astype(np.float32),    # f16 scale overflow -> inf
              (np.tile(np.arange(-7, 8), 9)[:g] * 2.0 ** -5).astype(np.float32),  # exact codes
              ((np.arange(g) % 14 - 7 + 0.5) * 2.0 ** -4).astype(np.float32)]     # ties
    groups[5][0] = np.float32(7 * 2.0 ** -4)
    nan = weights(33, (g,), 1.0)
    nan[5] = np.nan
    groups.append(nan)
    w = np.concatenate(groups)[None, :].repeat(3, axis=0)
    w = np.ascontiguousarray(w[:, : (w.shape[1] // g) * g])
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    rp, rs = oracle.quantize_i4_g128(w)
    assert np.array_equal(host(s).view(np.uint16), rs)
    assert np.array_equal(host(p), rp)
    assert ieee_equal(host(tq.dequantize_i4_g128(p, s)), oracle.dequantize_i4_g128(rp, rs))
    assert rs[0, 0] == 1 and rs[0, 2] == 1 and rs[0, 3] == 0x7C00


@pytest.mark.parametrize("shape", [(1, 128), (5, 384), (17, 1024), (3, 14336)])
def test_quantize_i4_g128_shapes(tq, oracle, shape):
    w = weights(34, shape)
    p, s = tq.quantize_i4_g128(dev_tensor(w))
    rp, rs = oracle.quantize_i4_g128(w)
    assert np.array_equal(host(s).view(np.uint16), rs) and np.array_equal(host(p), rp)
    assert ieee_equal(host(tq.dequantize_i4_g128(p, s)), oracle.dequantize_i4_g128(rp, rs))


# --------------------------------------------- generic reference primitives
def same_codes(gpu_f32, ref_f64):
    g = gpu_f32.astype(np.float64)
    return ieee_equal(g, ref_f64) and np.array_equal(np.signbit(g), np.signbit(ref_f64))


@pytest.mark.parametrize("dtype", [0, 1, 2, 3])
@pytest.mark.parametrize("scale,zp", [(0.01, 0.0), (1.0, 0.0), (0.0123, 3.0), (1.0 / 3.0, -2.0),
                                      (0.5, 0.0), (1e-10, 0.0), (0.0, 0.0)])
def test_quantize_tensor_matches_reference(tq, oracle, dtype, scale, zp):
    x = weights(40, (5000,), 1.0)
    x[:9] = [0.5, -0.5, 1.5, -2.5, -0.3, 0.0, -0.0, np.nan, np.inf]
    q = host(tq.quantize_tensor(dev_tensor(x), scale, zp, tq.QuantDType(dtype)))
    ref = oracle.quantize_tensor(x.astype(np.float64), scale, zp, dtype)
    assert same_codes(q, ref)
    d = host(tq.dequantize_tensor(dev_tensor(q), scale, zp))
    assert ieee_equal(d, oracle.dequantize_tensor(ref, scale, zp).astype(np.float32))
    f = host(tq.fake_quantize(dev_tensor(x), scale, zp, tq.QuantDType(dtype)))
    assert ieee_equal(f, oracle.fake_quantize(x.astype(np.float64), scale, zp, dtype).astype(np.float32))


def test_reference_unit_tests_through_api(tq):
    # quantize.rs:82-87, 89-99, 61-72, 101-136 restated on the GPU path
    q = host(tq.quantize_tensor([1000.0, -1000.0], 1.0, 0.0, tq.QuantDType.Int8))
    assert q.tolist() == [127.0, -128.0]
    r = host(tq.dequantize_tensor(np.array([0.0, 64.0, 127.0], np.float32), 0.01, 0.0))
    assert abs(r[0]) < 1e-7 and abs(r[1] - 0.64) < 1e-7 and abs(r[2] - 1.27) < 1e-7
    x = np.array([0.0, 0.5, 1.0, -0.5, -1.0], np.float32)
    q, s, z = tq.quantize_per_tensor(x, tq.QuantDType.Int8)
    d = host(tq.dequantize_tensor(q, s, z))
    assert np.all(np.abs(x - d) < 0.05)
    for dt, lo, hi in ((tq.QuantDType.Int4, -8, 7), (tq.QuantDType.UInt8, 0, 255)):
        q, _, _ = tq.quantize_per_tensor(np.array([0.0, 0.5, 1.0], np.float32), dt)
        q = host(q)
        assert q.shape == (3,) and np.all((q >= lo) & (q <= hi))
    f = tq.fake_quantize(np.ones((2, 3), np.float32), 0.1, 0.0, tq.QuantDType.Int8)
    assert tuple(f.shape) == (2, 3)


@pytest.mark.parametrize("dtype", [0, 1, 2, 3])
@pytest.mark.parametrize("n", [0, 1, 5, 1000, 1 << 20])
def test_quantize_per_tensor_matches_reference(tq, oracle, dtype, n):
    x = weights(41, (n,), 0.7) + 0.1
    q, s, z = tq.quantize_per_tensor(dev_tensor(x), tq.QuantDType(dtype))
    rq, rs, rz = oracle.quantize_per_tensor(x.astype(np.float64), dtype)
    assert (s, z) == (rs, rz)
    assert same_codes(host(q), rq)


def test_observers_match_reference(tq, oracle):
    o = tq.MinMaxObserver()
    ro = oracle.MinMaxObserver()
    assert o.compute_scale_zero_point(tq.QuantDType.Int8) == (1.0, 0.0)
    for seed in range(3):
        x = weights(42 + seed, (100000,), 1.0 + seed)
        x[seed] = np.nan
        o.observe(dev_tensor(x))
        ro.observe(x.astype(np.float64))
    assert (o.min_val(), o.max_val()) == (ro.min_val, ro.max_val)
    for dt in range(4):
        assert o.compute_scale_zero_point(tq.QuantDType(dt)) == ro.compute_scale_zero_point(dt)
    o.reset()
    assert (o.min_val(), o.max_val()) == (math.inf, -math.inf)

    pc = tq.PerChannelMinMaxObserver(37)
    rpc = oracle.PerChannelMinMaxObserver(37)
    x = weights(45, (37 * 300 + 5,), 1.0)  # trailing remainder ignored, as in the reference
    pc.observe(dev_tensor(x))
    rpc.observe(x.astype(np.float64))
    assert pc.min_vals() == rpc.mins.tolist() and pc.max_vals() == rpc.maxs.tolist()
    rs, rz = rpc.scales_and_zero_points(0)
    assert pc.scales_and_zero_points(tq.QuantDType.Int8) == list(zip(rs.tolist(), rz.tolist()))
    assert pc.compute_scale_zero_point(tq.QuantDType.Int8) == rpc.compute_scale_zero_point(0)


# ---------------------------------------- f64 data through the Python API
@pytest.mark.parametrize("dtype", [0, 1, 2, 3])
@pytest.mark.parametrize("scale,zp", [(0.01, 0.0), (1.0 / 3.0, -2.0), (0.0123, 3.0), (1e-300, 0.0)])
def test_python_api_f64_matches_reference(tq, oracle, dtype, scale, zp):
    """float64 tensors run the _f64 entry points: the reference's own element
    type, values that f32 cannot hold (x/scale within 2^-40 of a tie)."""
    import torch

    rng = np.random.default_rng(70 + dtype)
    x = rng.standard_normal(4000) * 3.0
    x[:8] = [2.5 * scale, -2.5 * scale, 0.5 * scale * (1 + 2.0 ** -40), -0.3 * scale, 0.0, -0.0, np.nan, -np.inf]
    xd = torch.from_numpy(x).cuda()
    q = tq.quantize_tensor(xd, scale, zp, tq.QuantDType(dtype))
    assert q.dtype == torch.float64
    ref = oracle.quantize_tensor(x, scale, zp, dtype)
    assert same_codes(host(q), ref)
    d = tq.dequantize_tensor(q, scale, zp)
    assert d.dtype == torch.float64 and ieee_equal(host(d), oracle.dequantize_tensor(ref, scale, zp))
    f = tq.fake_quantize(xd, scale, zp, tq.QuantDType(dtype))
    assert f.dtype == torch.float64 and ieee_equal(host(f), oracle.fake_quantize(x, scale, zp, dtype))
    q2, s2, z2 = tq.quantize_per_tensor(xd[8:], tq.QuantDType(dtype))
    rq2, rs2, rz2 = oracle.quantize_per_tensor(x[8:], dtype)
    assert (s2, z2) == (rs2, rz2) and same_codes(host(q2), rq2)


def test_observers_widen_to_f64(tq, oracle):
    """An f32 input, then f64 inputs whose extremes f32 cannot hold: the state
    widens exactly and keeps the reference's f64 min/max."""
    import torch

    o = tq.MinMaxObserver()
    ro = oracle.MinMaxObserver()
    x32 = weights(71, (1000,), 1.0)
    o.observe(dev_tensor(x32))
    ro.observe(x32.astype(np.float64))
    x64 = np.random.default_rng(72).standard_normal(3000) * 2.0
    x64[7] = 1.0 + 2.0 ** -40 + 9.0
    x64[8] = np.nan
    o.observe(torch.from_numpy(x64).cuda())
    ro.observe(x64)
    o.observe(dev_tensor(x32 * 0.5))
    ro.observe((x32 * 0.5).astype(np.float64))
    assert (o.min_val(), o.max_val()) == (ro.min_val, ro.max_val)
    for dt in range(4):
        assert o.compute_scale_zero_point(tq.QuantDType(dt)) == ro.compute_scale_zero_point(dt)
    pc = tq.PerChannelMinMaxObserver(11)
    rpc = oracle.PerChannelMinMaxObserver(11)
    x = np.random.default_rng(73).standard_normal(11 * 40) / 3.0
    pc.observe(torch.from_numpy(x).cuda())
    rpc.observe(x)
    assert pc.min_vals() == rpc.mins.tolist() and pc.max_vals() == rpc.maxs.tolist()
