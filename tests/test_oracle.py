"""Pins the C oracle (oracle/tq_oracle.c) before it is trusted as the checker.

Each group of tests names what pins the oracle function:
  * the reference's own unit-test asserts, restated (file:line cited);
  * exact rational arithmetic (fractions.Fraction) for the rounding rule;
  * independent library routines (numpy float16, torch bfloat16, numpy int64
    and f64 matmul) for conversions and products;
  * closed forms and brute force on small inputs.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

from conftest import ieee_equal

INT8, UINT8, INT4, FP8 = 0, 1, 2, 3


def rhaz(fr: Fraction) -> int:
    """round half away from zero of an exact rational."""
    a = abs(fr)
    n = math.floor(a + Fraction(1, 2))
    return n if fr >= 0 else -n


def exact_code(x: float, s: float, qmin: int, qmax: int) -> int:
    return max(qmin, min(qmax, rhaz(Fraction(float(x)) / Fraction(float(s)))))


# --------------------------------------------------------------- qconfig.rs
def test_qdtype_ranges_reference_asserts(oracle):
    # crates/theano-quantize/src/qconfig.rs:82-108
    assert [oracle.lib().tqo_bits(d) for d in (INT8, UINT8, INT4, FP8)] == [8, 8, 4, 8]
    assert [bool(oracle.lib().tqo_is_signed(d)) for d in (INT8, UINT8, INT4, FP8)] == [True, False, True, False]
    assert [oracle.lib().tqo_qmin(d) for d in (INT8, UINT8, INT4, FP8)] == [-128.0, 0.0, -8.0, -448.0]
    assert [oracle.lib().tqo_qmax(d) for d in (INT8, UINT8, INT4, FP8)] == [127.0, 255.0, 7.0, 448.0]


# -------------------------------------------------------------- quantize.rs
def test_quantize_tensor_clamps_kat(oracle):
    # quantize.rs:82-87
    q = oracle.quantize_tensor([1000.0, -1000.0], 1.0, 0.0, INT8)
    assert q.tolist() == [127.0, -128.0]


def test_dequantize_tensor_kat(oracle):
    # quantize.rs:89-99
    r = oracle.dequantize_tensor([0.0, 64.0, 127.0], 0.01, 0.0)
    assert len(r) == 3
    assert abs(r[0] - 0.0) < 1e-10 and abs(r[1] - 0.64) < 1e-10 and abs(r[2] - 1.27) < 1e-10


def test_quantize_dequantize_roundtrip_reference(oracle):
    # quantize.rs:61-72
    x = np.array([0.0, 0.5, 1.0, -0.5, -1.0])
    q, s, z = oracle.quantize_per_tensor(x, INT8)
    d = oracle.dequantize_tensor(q, s, z)
    assert np.all(np.abs(x - d) < 0.05)


def test_quantize_per_tensor_int4_uint8_ranges_reference(oracle):
    # quantize.rs:101-119
    q, _, _ = oracle.quantize_per_tensor([0.0, 0.5, 1.0], INT4)
    assert len(q) == 3 and np.all((q >= -8) & (q <= 7))
    q, _, _ = oracle.quantize_per_tensor([0.0, 0.5, 1.0], UINT8)
    assert np.all((q >= 0) & (q <= 255))


def test_quantize_single_value_reference(oracle):
    # quantize.rs:128-136
    q, s, z = oracle.quantize_per_tensor([0.5, -0.5], INT8)
    d = oracle.dequantize_tensor(q, s, z)
    assert abs(0.5 - d[0]) < 0.05 and abs(-0.5 - d[1]) < 0.05


def test_fake_quantize_shape_reference(oracle):
    # quantize.rs:74-79, 121-126 (shape preserved) + composition quantize->dequantize
    x = np.array([1.0, 2.0, 3.0, 4.0, 5.0, 6.0])
    f = oracle.fake_quantize(x, 0.1, 0.0, INT8)
    assert f.shape == x.shape
    q = oracle.quantize_tensor(x, 0.1, 0.0, INT8)
    assert np.array_equal(f, oracle.dequantize_tensor(q, 0.1, 0.0))


def test_quantize_per_tensor_closed_form(oracle):
    # quantize.rs:33-44 against the formula evaluated with exact rationals
    x = np.array([-0.75, -0.1, 0.0, 0.3, 1.25])
    q, s, z = oracle.quantize_per_tensor(x, UINT8)
    assert s == (1.25 - (-0.75)) / 255.0
    assert z == float(rhaz(Fraction(0.0) - Fraction(-0.75) / Fraction(s)))
    for xi, qi in zip(x, q):
        assert qi == max(0, min(255, rhaz(Fraction(float(xi)) / Fraction(s) + Fraction(z))))


def test_quantize_ties_half_away_from_zero(oracle):
    # Rust f64::round: halves go away from zero (numpy/torch round half to even)
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -127.5, -128.5, 127.5])
    q = oracle.quantize_tensor(x, 1.0, 0.0, INT8)
    assert q.tolist() == [1, 2, 3, -1, -2, -3, 127, -128, -128, 127]
    # x in (-s/2, 0) -> -0.0 code (sign kept), NaN propagates
    q = oracle.quantize_tensor([-0.3, float("nan")], 1.0, 0.0, INT8)
    assert q[0] == 0.0 and math.copysign(1.0, q[0]) == -1.0 and math.isnan(q[1])


def test_quantize_tensor_matches_exact_rationals(oracle):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal(20000) * 0.02).astype(np.float32).astype(np.float64)
    for s in (0.02 / 127, 1.0 / 3.0, 7.5e-4, float(np.float32(0.054 / 7))):
        q = oracle.quantize_tensor(x, s, 0.0, INT8)
        ref = [exact_code(v, s, -128, 127) for v in x]
        assert np.array_equal(q, ref)


# -------------------------------------------------------------- observer.rs
def test_minmax_observer_reference_asserts(oracle):
    o = oracle.MinMaxObserver()
    o.observe([1.0, 2.0, 3.0, -1.0])                      # observer.rs:142-148
    assert (o.min_val, o.max_val) == (-1.0, 3.0)
    o = oracle.MinMaxObserver()
    o.observe([1.0, 2.0])
    o.observe([-5.0, 10.0])                               # observer.rs:150-157
    assert (o.min_val, o.max_val) == (-5.0, 10.0)
    assert oracle.MinMaxObserver().compute_scale_zero_point(INT8) == (1.0, 0.0)  # :159-165
    o = oracle.MinMaxObserver()
    o.observe([0.0, 1.0])                                 # :167-174
    s, _ = o.compute_scale_zero_point(UINT8)
    assert abs(s - 1.0 / 255.0) < 1e-6
    o.reset()                                             # :176-186
    assert (o.min_val, o.max_val) == (math.inf, -math.inf)
    assert o.compute_scale_zero_point(INT8) == (1.0, 0.0)


def test_minmax_observer_ignores_nan(oracle):
    o = oracle.MinMaxObserver()
    o.observe([float("nan"), 2.0, -3.0, float("nan")])
    assert (o.min_val, o.max_val) == (-3.0, 2.0)


def test_per_channel_observer_reference_asserts(oracle):
    o = oracle.PerChannelMinMaxObserver(2)
    o.observe([1.0, 2.0, 3.0, -1.0, 0.0, 1.0])           # observer.rs:188-195
    s, z = o.scales_and_zero_points(INT8)
    assert len(s) == 2
    assert s[0] == (3.0 - 1.0) / 255.0 and s[1] == (1.0 - -1.0) / 255.0
    o = oracle.PerChannelMinMaxObserver(3)
    o.observe([1.0, 2.0, 3.0])
    o.reset()                                             # :197-206
    assert o.compute_scale_zero_point(INT8)[0] > 0.0
    o = oracle.PerChannelMinMaxObserver(2)
    o.observe([0.0, 1.0, 0.0, 2.0])                       # :215-223
    s, _ = o.compute_scale_zero_point(INT8)
    assert s > 0.0 and s == (1.0 / 255.0 + 2.0 / 255.0) / 2.0


# ---------------------------------------------------- f16 / bf16 conversions
def test_f64_to_f16_matches_numpy(oracle):
    rng = np.random.default_rng(5)
    vals = np.concatenate([
        rng.standard_normal(4000) * 0.01,
        rng.uniform(0, 1e-6, 2000),             # f16 subnormal range
        np.array([0.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 65504.0, 65519.99, 65520.0, 1e9,
                  (1 + 2 ** -11) * 1.0, (1 + 3 * 2 ** -11) * 1.0, 1e-10]),
    ])
    got = np.array([oracle.f64_to_f16_bits(v) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, ref)


def test_f16_decode_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float64)
    got = np.array([oracle.f16_bits_to_f64(int(b)) for b in bits])
    assert ieee_equal(got, ref)


def test_f32_to_bf16_matches_torch(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32),
                        np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -1.0 - 2 ** -8, 3.4e38], np.float32)])
    got = np.array([oracle.f32_to_bf16_bits(float(v)) for v in x], dtype=np.uint16)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


# ------------------------------------------------ build-defined INT8 per row
def test_quantize_i8_rowwise_exact(oracle):
    rng = np.random.default_rng(7)
    w = (rng.standard_normal((24, 300)) * 0.02).astype(np.float32)
    w[3, :] = 0.0                                   # zero row -> 1e-10 floor
    w[4, 5] = np.nan                                # NaN ignored by absmax, code 0
    q, s = oracle.quantize_i8_rowwise(w)
    for r in range(w.shape[0]):
        row = w[r]
        finite = row[~np.isnan(row)]
        absmax = float(np.max(np.abs(finite))) if finite.size else math.inf
        sc = np.float32(max(absmax / 127.0, 1e-10))
        assert s[r] == sc
        ref = [0 if np.isnan(v) else exact_code(v, sc, -128, 127) for v in row]
        assert q[r].tolist() == ref
    assert s[3] == np.float32(1e-10) and not q[3].any()
    d = oracle.dequantize_i8_rowwise(q, s)
    assert np.array_equal(d, (q.astype(np.float64) * s[:, None].astype(np.float64)).astype(np.float32))


def test_quantize_i8_rowwise_nonfinite_rows(oracle):
    w = np.array([[np.inf, 1.0, -2.0, 0.5], [np.nan] * 4, [-np.inf, 3.0, np.nan, -1.0]], np.float32)
    q, s = oracle.quantize_i8_rowwise(w)
    assert np.all(np.isinf(s)) and not q.any()  # x/inf = 0, inf/inf and NaN -> 0 (Rust `as`)


# ----------------------------------------------- build-defined INT4 group-128
def np_pack(codes):
    c = (codes.astype(np.int16) & 0xF).astype(np.uint8)
    return (c[:, 0::2] | (c[:, 1::2] << 4)).astype(np.uint8)


def test_quantize_i4_g128_exact(oracle):
    rng = np.random.default_rng(8)
    w = (rng.standard_normal((6, 512)) * 0.02).astype(np.float32)
    w[1, 128:256] = 0.0                       # zero group -> scale floor 2^-24
    w[2, 0:128] *= 1e-6                       # subnormal f16 scale
    p, s = oracle.quantize_i4_g128(w)
    codes = np.zeros(w.shape, np.int64)
    for r in range(w.shape[0]):
        for g in range(4):
            grp = w[r, g * 128:(g + 1) * 128]
            sf = np.float16(float(np.max(np.abs(grp))) / 7.0)
            if sf == 0:
                sf = np.uint16(1).view(np.float16)
            assert s[r, g] == sf.view(np.uint16)
            codes[r, g * 128:(g + 1) * 128] = [exact_code(v, float(sf), -8, 7) for v in grp]
    assert np.array_equal(p, np_pack(codes))
    assert s[1, 1] == 1
    d = oracle.dequantize_i4_g128(p, s)
    sc = s.view(np.float16).astype(np.float64).repeat(128, axis=1)
    assert np.array_equal(d, (codes * sc).astype(np.float32))


def test_int4_known_codes_and_nibble_order(oracle):
    # weights chosen so every code is known: group absmax = 7 * 2^-6
    q = np.tile(np.arange(-7, 8), 10)[:128].astype(np.int64)
    q[0] = 7
    w = (q * 2.0 ** -6).astype(np.float32)[None, :]
    p, s = oracle.quantize_i4_g128(w)
    assert s[0, 0] == np.float16(2.0 ** -6).view(np.uint16)
    assert p[0, 0] == ((7 & 0xF) | ((-6 & 0xF) << 4))  # low nibble = even k
    assert np.array_equal(p, np_pack(q[None, :]))


def test_int4_pack_unpack_bijection(oracle):
    allbytes = np.arange(256, dtype=np.uint8)
    p = np.tile(allbytes, 1).reshape(4, 64)           # 4 rows of K=128
    s = np.full((4, 1), np.float16(1.0).view(np.uint16), np.uint16)
    codes = oracle.dequantize_i4_g128(p, s).astype(np.int64)
    assert codes.min() == -8 and codes.max() == 7
    assert np.array_equal(np_pack(codes), p)


# ------------------------------------------------------------ mm / Linear
def test_mm_reference_kats(oracle):
    a = np.array([[1.0, 2.0, 3.0], [4.0, 5.0, 6.0]])
    b = np.array([[7.0, 8.0], [9.0, 10.0], [11.0, 12.0]])
    assert oracle.mm(a, b).ravel().tolist() == [58.0, 64.0, 139.0, 154.0]   # tensor_ops.rs:841-849
    assert oracle.mm(a[:1], b).ravel().tolist() == [58.0, 64.0]              # :853-859
    assert oracle.mm([[1.0, 2.0, 3.0]], [[4.0], [5.0], [6.0]])[0, 0] == 32.0  # :863+ dot


def test_mm_vs_numpy(oracle):
    rng = np.random.default_rng(9)
    a = rng.integers(-50, 50, (7, 33)).astype(np.float64)
    b = rng.integers(-50, 50, (33, 5)).astype(np.float64)
    assert np.array_equal(oracle.mm(a, b), a @ b)           # exact on integers
    a = rng.standard_normal((9, 70))
    b = rng.standard_normal((70, 11))
    np.testing.assert_allclose(oracle.mm(a, b), a @ b, rtol=1e-12, atol=1e-12)


def test_mm_sequential_k_order(oracle):
    # i-p-j accumulates p in order: (1e16 + 1) - 1e16 = 0 in f64, not 1
    a = np.array([[1.0, 1.0, 1.0]])
    b = np.array([[1e16], [1.0], [-1e16]])
    assert oracle.mm(a, b)[0, 0] == 0.0


def test_linear_bias_and_transpose(oracle):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((3, 6))
    w = rng.standard_normal((4, 6))
    b = rng.standard_normal(4).astype(np.float32)
    np.testing.assert_allclose(oracle.linear(x, w, b), x @ w.T + b.astype(np.float64), rtol=1e-12, atol=1e-12)


def test_linear_w8_w4_match_numpy(oracle):
    rng = np.random.default_rng(12)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    x = rng.standard_normal((3, 256)).astype(np.float32)
    q, s = oracle.quantize_i8_rowwise(w)
    ref = x.astype(np.float64) @ (q.astype(np.float64) * s[:, None].astype(np.float64)).T
    np.testing.assert_allclose(oracle.linear_w8(x, q, s), ref, rtol=1e-12, atol=1e-12)
    p, s16 = oracle.quantize_i4_g128(w)
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)         # truncation: any bf16 pattern will do
    xf = (xb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    wd = oracle.dequantize_i4_g128(p, s16).astype(np.float64)
    np.testing.assert_allclose(oracle.linear_w4g128_bf16(xb, p, s16), xf @ wd.T, rtol=1e-12, atol=1e-12)


def test_linear_w4g128_f32_and_bias_match_numpy(oracle):
    """Linear::forward over the dequantized INT4 weight with f32 activations
    (linear.rs:111-121 over quantize.rs:22-27): x @ deq(W)^T + b in f64.  The
    activations are not multiples of a bf16 ulp, so a path that rounded them to
    bf16 fails; distinct row/column sizes and a bias catch a swapped argument."""
    rng = np.random.default_rng(15)
    n, k, m = 40, 384, 3
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    p, s16 = oracle.quantize_i4_g128(w)
    wd = oracle.dequantize_i4_g128(p, s16).astype(np.float64)
    ref = x.astype(np.float64) @ wd.T
    got = oracle.linear_w4g128_f32(x, p, s16)
    assert got.shape == (m, n)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(oracle.linear_w4g128_f32(x, p, s16, b), ref + b.astype(np.float64), rtol=1e-12,
                               atol=1e-12)
    # the f32 values reach the sum unrounded: the bf16 form of the same x differs
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.abs(oracle.linear_w4g128_bf16(xb, p, s16) - got).max() > 1e-6
    # a row of the product is the sequential f64 dot of Tensor::mm (tensor_ops.rs:379-410)
    acc = 0.0
    for kk in range(k):
        acc += float(x[1, kk]) * float(wd[7, kk])
    assert got[1, 7] == pytest.approx(acc, rel=1e-13, abs=1e-15)


# ------------------------------------------------------------------ W8A8
def test_w8a8_acc_vs_numpy_int64(oracle):
    rng = np.random.default_rng(13)
    qa = rng.integers(-128, 128, (9, 320)).astype(np.int8)
    qw = rng.integers(-128, 128, (7, 320)).astype(np.int8)
    acc = oracle.gemm_w8a8_acc(qa, qw)
    assert np.array_equal(acc, qa.astype(np.int64) @ qw.astype(np.int64).T)
    ext = np.full((2, 4096), -128, np.int8)                   # |acc| extreme: 4096*128*128 = 2^26
    assert oracle.gemm_w8a8_acc(ext, ext)[0, 0] == 4096 * 128 * 128


def test_linear_w8a8_vs_numpy(oracle):
    rng = np.random.default_rng(14)
    qa = rng.integers(-127, 128, (5, 128)).astype(np.int8)
    qw = rng.integers(-127, 128, (6, 128)).astype(np.int8)
    sa = rng.uniform(0.001, 0.01, 5).astype(np.float32)
    sw = rng.uniform(0.001, 0.01, 6).astype(np.float32)
    ref = (qa * sa[:, None].astype(np.float64)) @ (qw * sw[:, None].astype(np.float64)).T
    np.testing.assert_allclose(oracle.linear_w8a8(qa, sa, qw, sw), ref, rtol=1e-12, atol=1e-15)


# ------------------------------------------------------------- SiLU / MLP
def test_sigmoid_silu_closed_forms(oracle):
    assert oracle.sigmoid(0.0) == 0.5
    assert oracle.silu_module(0.0) == 0.0
    assert oracle.silu_module(40.0) == 40.0
    assert oracle.silu_module(-800.0) == 0.0      # exp overflow -> 1/inf -> -0
    assert abs(oracle.silu_module(1.0) - 1.0 / (1.0 + math.e ** -1.0)) < 1e-15


def test_mlp_matches_numpy_composition(oracle):
    rng = np.random.default_rng(15)
    d, f, m = 256, 384, 3
    wg = (rng.standard_normal((f, d)) * 0.02).astype(np.float32)
    wu = (rng.standard_normal((f, d)) * 0.02).astype(np.float32)
    wd = (rng.standard_normal((d, f)) * 0.02).astype(np.float32)
    x = (rng.standard_normal((m, d)).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    pg, sg = oracle.quantize_i4_g128(wg)
    pu, su = oracle.quantize_i4_g128(wu)
    pd, sd = oracle.quantize_i4_g128(wd)
    y = oracle.mlp_w4g128(x, pg, sg, pu, su, pd, sd)
    xf = (x.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    g = xf @ oracle.dequantize_i4_g128(pg, sg).astype(np.float64).T
    u = xf @ oracle.dequantize_i4_g128(pu, su).astype(np.float64).T
    h = g * (1.0 / (1.0 + np.exp(-g))) * u
    ref = h @ oracle.dequantize_i4_g128(pd, sd).astype(np.float64).T
    np.testing.assert_allclose(y, ref, rtol=1e-11, atol=1e-12)


# ------------------------------------------------------------- FP8 (OCP e4m3)
# torch.float8_e4m3fn is an independent implementation of the same OCP format.
def _torch_e4m3(x):
    import torch

    return torch.from_numpy(np.asarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _torch_decode(codes):
    import torch

    return torch.from_numpy(np.asarray(codes, np.uint8)).view(torch.float8_e4m3fn).to(torch.float32).numpy()


def _e4m3_probe_values():
    finite = _torch_decode(np.arange(256, dtype=np.uint8))
    grid = np.unique(finite[np.isfinite(finite) & (finite >= 0)].astype(np.float64))
    grid = np.append(grid, 480.0)  # one step past 448: the rounding boundary at 464
    mids = (grid[:-1] + grid[1:]) / 2  # every tie, exact in f32
    pts = np.concatenate([grid, mids]).astype(np.float32)
    up = np.nextafter(pts, np.float32(np.inf))
    dn = np.nextafter(pts, np.float32(-np.inf))
    rng = np.random.default_rng(7)
    wide = (rng.standard_normal(20000) * np.exp2(rng.uniform(-14, 10, 20000))).astype(np.float32)
    special = np.array([0.0, 2.0 ** -10, 2.0 ** -11, 1e-30, 1e-45, 447.9, 448.0, 463.99, 464.0, 464.01, 479.0,
                        480.0, 500.0, 1e30, np.inf, np.nan], np.float32)
    v = np.concatenate([pts, up, dn, wide, special])
    return np.concatenate([v, -v])


def test_e4m3_decode_all_codes_vs_torch(oracle):
    t = _torch_decode(np.arange(256, dtype=np.uint8)).astype(np.float64)
    o = np.array([oracle.e4m3_to_f64(c) for c in range(256)])
    assert ieee_equal(o, t)
    # format facts: 0x7E = 448, 0x08 = 2^-6 (smallest normal), 0x01 = 2^-9, NaN only at S.1111.111
    assert o[0x7E] == 448.0 and o[0x08] == 2.0 ** -6 and o[0x01] == 2.0 ** -9 and o[0x38] == 1.0
    assert [c for c in range(256) if math.isnan(o[c])] == [0x7F, 0xFF]


def test_e4m3_encode_vs_torch(oracle):
    v = _e4m3_probe_values()
    o = np.array([oracle.f32_to_e4m3(float(x)) for x in v], np.uint8)
    assert np.array_equal(o, _torch_e4m3(v))


def test_e4m3_encode_ties_to_even_and_overflow(oracle):
    f = oracle.f32_to_e4m3
    assert f(1.0625) == 0x38          # tie between 1 and 1.125 -> even mantissa (1.0)
    assert f(1.1875) == 0x3A          # tie between 1.125 and 1.25 -> 1.25
    assert f(3 * 2.0 ** -10) == 0x02  # subnormal tie between 1 and 2 (x 2^-9) -> 2
    assert f(2.0 ** -10) == 0x00 and f(-(2.0 ** -10)) == 0x80
    assert f(464.0) == 0x7E and f(464.01) == 0x7F and f(-500.0) == 0xFF
    assert f(float("inf")) == 0x7F and f(float("-inf")) == 0xFF


def _f32(x):
    return float(np.float32(x))


def test_quantize_fp8_rowwise_exact(oracle):
    rng = np.random.default_rng(11)
    w = (rng.standard_normal((6, 300)) * np.exp2(rng.uniform(-8, 8, (6, 1)))).astype(np.float32)
    w[1, 17] = -abs(w[1]).max() * 2  # the absmax element negative
    w[2, :] = 0.0
    w[3, 5] = np.nan
    w[4, 9] = np.inf
    w[5, 0] = -0.0
    q, s = oracle.quantize_fp8_rowwise(w)
    dec = _torch_decode(q).astype(np.float64)
    for r in range(w.shape[0]):
        row = w[r].astype(np.float64)
        absmax = np.nanmax(np.abs(row))
        # scale: f32 of the f64 quotient absmax / 448, floored at 1e-10
        assert s[r] == np.float32(max(absmax / 448.0, 1e-10))
        for i, x in enumerate(row):
            if math.isnan(x) or (math.isinf(x) and math.isinf(s[r])):
                assert q[r, i] == 0x7F
                continue
            qt = _f32(Fraction(x) / Fraction(float(s[r]))) if math.isfinite(s[r]) else 0.0 * x
            # the code is a nearest e4m3 value of the f32 quotient (clamped to +-448)
            c = dec[r, i]
            t = max(-448.0, min(448.0, qt))
            grid_step = 2.0 ** (max(math.floor(math.log2(abs(t))), -6) - 3) if t != 0 else 2.0 ** -9
            assert abs(c - t) <= grid_step / 2, (r, i, x, c, t)
            assert (q[r, i] >> 7) == int(math.copysign(1.0, x) < 0), (r, i, x)  # sign bit of x, zeros too
    assert q[2].tolist() == [0] * 300 and s[2] == np.float32(1e-10)
    assert q[5, 0] == 0x80                         # -0 keeps its sign
    assert np.all(q[4, np.arange(300) != 9] & 0x7F == 0)  # finite / inf -> +-0
    # the absmax element lands on +-448
    assert q[1, 17] == 0xFE and np.abs(dec[0]).max() == 448.0


def test_quantize_fp8_rowwise_vs_torch_composition(oracle):
    import torch

    rng = np.random.default_rng(12)
    w = (rng.standard_normal((16, 512)) * 3).astype(np.float32)
    q, s = oracle.quantize_fp8_rowwise(w)
    s_ref = np.maximum(np.abs(w.astype(np.float64)).max(axis=1) / 448.0, 1e-10).astype(np.float32)
    assert np.array_equal(s, s_ref)
    t = torch.from_numpy(w) / torch.from_numpy(s_ref)[:, None]
    ref = t.clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(q, ref)


def test_dequantize_fp8_rowwise_vs_numpy(oracle):
    rng = np.random.default_rng(13)
    q = rng.integers(0, 256, (5, 64), dtype=np.uint8)
    s = (rng.uniform(0.5, 2, 5) * np.exp2(rng.integers(-20, 20, 5))).astype(np.float32)
    out = oracle.dequantize_fp8_rowwise(q, s)
    ref = _torch_decode(q) * s[:, None]  # f32 product: one rounding
    assert ieee_equal(out, ref)


def test_linear_fp8_vs_numpy(oracle):
    rng = np.random.default_rng(14)
    qa = rng.integers(0, 256, (7, 96), dtype=np.uint8)
    qw = rng.integers(0, 256, (9, 96), dtype=np.uint8)
    qa[(qa & 0x7F) == 0x7F] = 0x38
    qw[(qw & 0x7F) == 0x7F] = 0xB8
    sa = rng.uniform(0.5, 2, 7).astype(np.float32)
    sw = rng.uniform(0.5, 2, 9).astype(np.float32)
    b = rng.standard_normal(9).astype(np.float32)
    a = _torch_decode(qa).astype(np.float64) * sa[:, None].astype(np.float64)
    w = _torch_decode(qw).astype(np.float64) * sw[:, None].astype(np.float64)
    ref = a @ w.T + b.astype(np.float64)
    y = oracle.linear_fp8(qa, sa, qw, sw, b)
    assert np.allclose(y, ref, rtol=1e-12, atol=1e-9)


# ------------------------------------------------------ element conversion
DT_F16, DT_BF16, DT_F32, DT_F64, DT_U8, DT_I8, DT_I16, DT_I32, DT_I64, DT_BOOL = range(10)


def conversion_probe_f64():
    """f64 values around every rounding case of the narrow float types."""
    rng = np.random.default_rng(21)
    wide = rng.standard_normal(3000) * np.exp2(rng.uniform(-160, 130, 3000))
    f32_ties = (np.float32(rng.standard_normal(500)).astype(np.float64) +
                np.spacing(np.float32(1)).astype(np.float64) * 0)  # exact f32 values
    half_ulp = np.spacing(np.abs(f32_ties).astype(np.float32)).astype(np.float64) / 2
    ties = np.concatenate([f32_ties + half_ulp, f32_ties - half_ulp])
    near = np.nextafter(ties, np.inf)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65520.0, 65519.99, 2.0 ** -24, 2.0 ** -25,
                        3 * 2.0 ** -26, 3.4e38, 3.4028235677973366e38, 3.402823669209385e38, 1e-45, 2.0 ** -149,
                        2.0 ** -150, 3 * 2.0 ** -151, 2.0 ** -133, 2.0 ** -134, 3 * 2.0 ** -135, 1e-320,
                        127.5, 128.0, -128.5, -129.0, 255.5, 256.0, -0.7, 2.0 ** 31, -(2.0 ** 31) - 0.5,
                        2.0 ** 63, -(2.0 ** 63), 9.2e18, -9.2e18, 2.0 ** 53 + 1, 1e300])
    return np.concatenate([wide, ties, near, special, -special])


def test_dtype_sizes_reference_asserts(oracle):
    # crates/theano-types/src/dtype.rs:107-114
    sz = {n: oracle.lib().tqo_dtype_size(i) for i, n in enumerate(oracle.DTYPES)}
    assert sz["float32"] == 4 and sz["float64"] == 8 and sz["float16"] == 2 and sz["bfloat16"] == 2
    assert sz["int64"] == 8 and sz["bool"] == 1
    assert [sz[n] for n in ("uint8", "int8", "int16", "int32")] == [1, 1, 2, 4]
    assert oracle.lib().tqo_dtype_size(10) == 0


def test_convert_f64_to_f32_f16_vs_numpy(oracle):
    v = conversion_probe_f64()
    got32 = oracle.convert(v, DT_F64, DT_F32)
    assert ieee_equal(got32, v.astype(np.float32)) and np.array_equal(np.signbit(got32), np.signbit(v))
    got16 = oracle.convert(v, DT_F64, DT_F16).view(np.float16)
    ref16 = v.astype(np.float16)
    assert ieee_equal(got16, ref16) and np.array_equal(np.signbit(got16), np.signbit(ref16))


def _bf16_exact(x):
    """Nearest bf16 (ties to even) of a finite f64 by exact rationals over all bf16 values."""
    if x != x:
        return None
    allv = np.arange(0, 0x7F81, dtype=np.uint32)  # +0 .. +inf
    vals = (allv << 16).view(np.float32).astype(np.float64)
    a = abs(x)
    i = int(np.searchsorted(vals, a))
    if i < len(vals) and vals[i] == a:
        code = int(allv[i])
    else:
        lo, hi = i - 1, i
        if hi == len(vals) - 1:  # between max finite and inf: inf past the midpoint to 2^128
            mid = (Fraction(vals[lo]) + Fraction(2) ** 128) / 2
            code = 0x7F80 if Fraction(a) >= mid else int(allv[lo])
        else:
            dl, dh = Fraction(a) - Fraction(vals[lo]), Fraction(vals[hi]) - Fraction(a)
            code = int(allv[lo]) if dl < dh or (dl == dh and allv[lo] % 2 == 0) else int(allv[hi])
    return code | (0x8000 if math.copysign(1.0, x) < 0 else 0)


def test_convert_f64_to_bf16_exact(oracle):
    v = conversion_probe_f64()[::7]
    got = oracle.convert(v, DT_F64, DT_BF16)
    for x, g in zip(v, got):
        ref = _bf16_exact(float(x))
        if ref is None:
            assert (g & 0x7F80) == 0x7F80 and (g & 0x7F) != 0
        else:
            assert g == ref, (x, hex(g), hex(ref))


def test_convert_float_to_int_rust_as(oracle):
    v = np.array([0.0, -0.0, 0.7, -0.7, 127.9, 128.0, -128.9, -129.0, 255.5, 256.0, -1.0, np.nan, np.inf,
                  -np.inf, 2.0 ** 31, -(2.0 ** 31) - 0.5, 2.0 ** 63, -(2.0 ** 63), 9.2e18, -9.2e18, 1e300, 3e4,
                  -4e4])
    i8 = oracle.convert(v, DT_F64, DT_I8).tolist()
    assert i8[:12] == [0, 0, 0, 0, 127, 127, -128, -128, 127, 127, -1, 0] and i8[12:14] == [127, -128]
    u8 = oracle.convert(v, DT_F64, DT_U8).tolist()
    assert u8[:13] == [0, 0, 0, 0, 127, 128, 0, 0, 255, 255, 0, 0, 255] and u8[13] == 0
    i32 = oracle.convert(v, DT_F64, DT_I32).tolist()
    assert i32[14:16] == [2 ** 31 - 1, -(2 ** 31)]
    i64 = oracle.convert(v, DT_F64, DT_I64).tolist()
    assert i64[16:20] == [2 ** 63 - 1, -(2 ** 63), 9200000000000000000, -9200000000000000000]
    assert i64[11] == 0 and i64[12] == 2 ** 63 - 1 and i64[13] == -(2 ** 63)
    i16 = oracle.convert(v, DT_F64, DT_I16).tolist()
    assert i16[21:] == [30000, -32768]
    b = oracle.convert(v, DT_F64, DT_BOOL).tolist()
    assert b[:4] == [0, 0, 1, 1] and b[11] == 1  # NaN != 0


def test_convert_sources_decode_exactly(oracle):
    h = np.arange(0, 65536, 17, dtype=np.uint16)
    assert ieee_equal(oracle.convert(h, DT_F16, DT_F64), h.view(np.float16).astype(np.float64))
    assert ieee_equal(oracle.convert(h, DT_BF16, DT_F64), (h.astype(np.uint32) << 16).view(np.float32).astype(np.float64))
    big = np.array([2 ** 53 + 1, -(2 ** 63), 2 ** 63 - 1, 12345], dtype=np.int64)
    assert np.array_equal(oracle.convert(big, DT_I64, DT_F64), big.astype(np.float64))  # RNE above 2^53
    assert oracle.convert(np.array([0, 1, 7], np.uint8), DT_BOOL, DT_F32).tolist() == [0.0, 1.0, 1.0]


# ------------------------------------------------ attention (transformer.rs)
def _np_attention(q, k, v, heads, mask=None):
    B, S, E = q.shape
    D = E // heads
    qh = q.reshape(B, S, heads, D).transpose(0, 2, 1, 3)
    kh = k.reshape(B, S, heads, D).transpose(0, 2, 1, 3)
    vh = v.reshape(B, S, heads, D).transpose(0, 2, 1, 3)
    sc = qh @ kh.transpose(0, 1, 3, 2) * (1.0 / math.sqrt(D))
    if mask is not None:
        sc = sc + mask.reshape(mask.shape[0], 1, S, S)
    with np.errstate(invalid="ignore"):
        e = np.exp(sc - sc.max(axis=-1, keepdims=True))
        p = e / e.sum(axis=-1, keepdims=True)
    return (p @ vh).transpose(0, 2, 1, 3).reshape(B, S, E)


def test_attention_closed_forms(oracle):
    rng = np.random.default_rng(31)
    B, S, H, D = 2, 5, 2, 3
    q = rng.standard_normal((B, S, H * D))
    v = rng.standard_normal((B, S, H * D))
    k = np.repeat(rng.standard_normal((B, 1, H * D)), S, axis=1)  # identical keys: uniform weights
    out = oracle.attention(q, k, v, H)
    assert np.allclose(out, np.repeat(v.mean(axis=1, keepdims=True), S, axis=1), rtol=1e-12, atol=1e-14)
    # causal mask (transformer.rs:238-246): the first query sees only the first key
    mask = np.triu(np.full((1, S, S), -np.inf), k=1)
    out = oracle.attention(q, rng.standard_normal((B, S, H * D)), v, H, mask)
    assert np.array_equal(out[:, 0], v[:, 0])
    # a row masked everywhere is NaN (softmax of -inf row), others are finite
    mask = np.zeros((B, S, S))
    mask[1, 2, :] = -np.inf
    out = oracle.attention(q, k, v, H, mask)
    assert np.isnan(out[1, 2]).all() and np.isfinite(np.delete(out[1], 2, axis=0)).all()


def test_attention_matches_numpy(oracle):
    rng = np.random.default_rng(32)
    B, S, H, D = 2, 9, 4, 8
    q, k, v = (rng.standard_normal((B, S, H * D)) for _ in range(3))
    mask = np.where(rng.random((B, S, S)) < 0.3, -np.inf, rng.standard_normal((B, S, S)))
    mask[:, :, 0] = 0.0  # at least one key per row
    for m in (None, mask, mask[:1]):
        assert np.allclose(oracle.attention(q, k, v, H, m), _np_attention(q, k, v, H, m), rtol=1e-12, atol=1e-13)
    # one head spanning the whole embedding
    assert np.allclose(oracle.attention(q, k, v, 1), _np_attention(q, k, v, 1), rtol=1e-12, atol=1e-13)
