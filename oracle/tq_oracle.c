/*
 * tq_oracle.c -- CPU restatement of neo-theano's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for libtq.so (see tq_oracle.h
 * for who may use it and how each function is pinned).  Compile with
 * -O2 -ffp-contract=off and without -ffast-math so that every double
 * operation rounds exactly like the reference's Rust f64 code.
 *
 * Citations are relative to the reference repository root.
 */
#include "tq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---- QuantDType ranges: crates/theano-quantize/src/qconfig.rs:12-41 ---- */

int tqo_bits(int dtype) { return dtype == TQO_INT4 ? 4 : 8; }

int tqo_is_signed(int dtype) { return dtype == TQO_INT8 || dtype == TQO_INT4; }

double tqo_qmin(int dtype) {
    switch (dtype) {
    case TQO_INT8: return -128.0;
    case TQO_UINT8: return 0.0;
    case TQO_INT4: return -8.0;
    default: return -448.0; /* FP8: range only, no encoding */
    }
}

double tqo_qmax(int dtype) {
    switch (dtype) {
    case TQO_INT8: return 127.0;
    case TQO_UINT8: return 255.0;
    case TQO_INT4: return 7.0;
    default: return 448.0;
    }
}

/* Rust f64::clamp: below min -> min, above max -> max, NaN passes through. */
static double rust_clamp(double x, double lo, double hi) {
    if (x < lo) x = lo;
    if (x > hi) x = hi;
    return x;
}

/* Rust `f64 as i8/i32`: NaN -> 0, otherwise truncate and saturate. */
static int32_t rust_as_int(double x, double lo, double hi) {
    if (x != x) return 0;
    if (x < lo) return (int32_t)lo;
    if (x > hi) return (int32_t)hi;
    return (int32_t)x;
}

/* ---- quantize.rs:8-19 quantize_tensor: q = round(x/scale + zp).clamp(qmin, qmax) ---- */
void tqo_quantize_tensor(const double* x, int64_t n, double scale, double zero_point,
                         int dtype, double* q) {
    const double qmin = tqo_qmin(dtype), qmax = tqo_qmax(dtype);
    for (int64_t i = 0; i < n; ++i)
        q[i] = rust_clamp(round(x[i] / scale + zero_point), qmin, qmax);
}

/* ---- quantize.rs:22-27 dequantize_tensor: x = (q - zp) * scale ---- */
void tqo_dequantize_tensor(const double* q, int64_t n, double scale, double zero_point,
                           double* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = (q[i] - zero_point) * scale;
}

/* ---- quantize.rs:30-48 quantize_per_tensor (asymmetric, stats from the data) ---- */
void tqo_quantize_per_tensor(const double* x, int64_t n, int dtype, double* q,
                             double* scale_out, double* zp_out) {
    double mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) mn = fmin(mn, x[i]);
    for (int64_t i = 0; i < n; ++i) mx = fmax(mx, x[i]);
    const double qmin = tqo_qmin(dtype), qmax = tqo_qmax(dtype);
    const double scale = fmax((mx - mn) / (qmax - qmin), 1e-10);
    const double zp = rust_clamp(round(qmin - mn / scale), qmin, qmax);
    for (int64_t i = 0; i < n; ++i) q[i] = rust_clamp(round(x[i] / scale + zp), qmin, qmax);
    *scale_out = scale;
    *zp_out = zp;
}

/* ---- quantize.rs:51-55 fake_quantize = dequantize(quantize(x)) ---- */
void tqo_fake_quantize(const double* x, int64_t n, double scale, double zero_point,
                       int dtype, double* out) {
    tqo_quantize_tensor(x, n, scale, zero_point, dtype, out);
    tqo_dequantize_tensor(out, n, scale, zero_point, out);
}

/* ---- observer.rs:42-73 MinMaxObserver ---- */
void tqo_minmax_observe(double* st, const double* values, int64_t n) {
    for (int64_t i = 0; i < n; ++i) {
        st[0] = fmin(st[0], values[i]);
        st[1] = fmax(st[1], values[i]);
    }
    st[2] = 1.0;
}

static void scale_zp_from_range(double mn, double mx, int dtype, double* scale, double* zp) {
    const double qmin = tqo_qmin(dtype), qmax = tqo_qmax(dtype);
    double s = (mx - mn) / (qmax - qmin);
    s = fmax(s, 1e-10);
    double z = qmin - mn / s;
    *scale = s;
    *zp = rust_clamp(round(z), qmin, qmax);
}

void tqo_minmax_scale_zp(const double* st, int dtype, double* scale, double* zp) {
    if (st[2] == 0.0) {
        *scale = 1.0;
        *zp = 0.0;
        return;
    }
    scale_zp_from_range(st[0], st[1], dtype, scale, zp);
}

/* ---- observer.rs:93-136 PerChannelMinMaxObserver (layout [channels, ...]) ---- */
void tqo_perchannel_observe(double* mins, double* maxs, int64_t channels,
                            const double* values, int64_t n) {
    const int64_t per = n / channels;
    for (int64_t c = 0; c < channels; ++c)
        for (int64_t i = 0; i < per; ++i) {
            const double v = values[c * per + i];
            mins[c] = fmin(mins[c], v);
            maxs[c] = fmax(maxs[c], v);
        }
}

void tqo_perchannel_scales_zps(const double* mins, const double* maxs, int64_t channels,
                               int dtype, double* scales, double* zps) {
    for (int64_t c = 0; c < channels; ++c)
        scale_zp_from_range(mins[c], maxs[c], dtype, &scales[c], &zps[c]);
}

void tqo_perchannel_global_scale_zp(const double* mins, const double* maxs,
                                    int64_t channels, int dtype, double* scale, double* zp) {
    double ss = 0.0, zz = 0.0;
    for (int64_t c = 0; c < channels; ++c) {
        double s, z;
        scale_zp_from_range(mins[c], maxs[c], dtype, &s, &z);
        ss += s;
        zz += z;
    }
    *scale = ss / (double)channels;
    *zp = zz / (double)channels;
}

/* ---- tensor_ops.rs:379-410 Tensor::mm: C[i,j] += A[i,p]*B[p,j], i-p-j order ---- */
void tqo_mm(const double* a, const double* b, int64_t m, int64_t k, int64_t n, double* c) {
    memset(c, 0, sizeof(double) * (size_t)(m * n));
    for (int64_t i = 0; i < m; ++i)
        for (int64_t p = 0; p < k; ++p) {
            const double av = a[i * k + p];
            const double* brow = b + p * n;
            double* crow = c + i * n;
            for (int64_t j = 0; j < n; ++j) crow[j] += av * brow[j];
        }
}

/* ---- linear.rs:111-121 Linear::forward: y = x . W^T (+ b) ----
 * W^T is materialised the way Tensor::mm's to_vec_f64 gathers the transposed
 * view (tensor_view.rs:129-163, tensor_ops.rs:395-396); the bias add is the
 * broadcast binary_op (tensor_ops.rs:125-147). */
void tqo_linear(const double* x, int64_t m, const double* w, const float* bias,
                int64_t n, int64_t k, double* y) {
    double* wt = (double*)malloc(sizeof(double) * (size_t)(n * k));
    for (int64_t p = 0; p < k; ++p)
        for (int64_t j = 0; j < n; ++j) wt[p * n + j] = w[j * k + p];
    tqo_mm(x, wt, m, k, n, y);
    free(wt);
    if (bias)
        for (int64_t i = 0; i < m; ++i)
            for (int64_t j = 0; j < n; ++j) y[i * n + j] = y[i * n + j] + (double)bias[j];
}

/* tensor_ops.rs:62-64 sigmoid = 1/(1+exp(-x)); activation.rs:70-74 SiLU = x*sigmoid(x) */
double tqo_sigmoid(double x) { return 1.0 / (1.0 + exp(-x)); }

double tqo_silu_module(double x) { return x * tqo_sigmoid(x); }

/* ---- IEEE round-to-nearest-even conversions for the build-defined formats ---- */
uint16_t tqo_f64_to_f16_bits(double x) {
    const uint16_t sign = signbit(x) ? 0x8000u : 0u;
    if (x != x) return (uint16_t)(sign | 0x7E00u);
    const double a = fabs(x);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u); /* past max + half ulp */
    if (a < 0x1p-14) {                                    /* subnormal range, ulp 2^-24 */
        const double m = nearbyint(a * 0x1p24);           /* exact scaling, RNE */
        return (uint16_t)(sign | (uint16_t)m);            /* m == 1024 encodes 2^-14 */
    }
    int e2;
    frexp(a, &e2);
    int e = e2 - 1; /* a in [2^e, 2^(e+1)) */
    double m = nearbyint(ldexp(a, 10 - e));
    if (m == 2048.0) {
        m = 1024.0;
        e += 1;
    }
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)(m - 1024.0));
}

double tqo_f16_bits_to_f64(uint16_t h) {
    const double sign = (h & 0x8000u) ? -1.0 : 1.0;
    const int e = (h >> 10) & 0x1F;
    const int m = h & 0x3FF;
    if (e == 0x1F) return m ? NAN : sign * INFINITY;
    if (e == 0) return sign * ldexp((double)m, -24);
    return sign * ldexp((double)(m + 1024), e - 25);
}

uint16_t tqo_f32_to_bf16_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

double tqo_bf16_bits_to_f64(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return (double)f;
}

/* ---- build-defined: symmetric absmax from the observer statistics ----
 * absmax = max(|min|, |max|) with min/max folded as in
 * PerChannelMinMaxObserver::observe (observer.rs:110-121).  A row with no
 * non-NaN value keeps min=+inf, max=-inf, so absmax = +inf. */
static double absmax_of(const float* v, int64_t n) {
    double mn = INFINITY, mx = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        mn = fmin(mn, (double)v[i]);
        mx = fmax(mx, (double)v[i]);
    }
    return fmax(fabs(mn), fabs(mx));
}

/* Build-defined symmetric per-row INT8:
 *   s_r = f32(max(absmax_r / 127, 1e-10))            (the 1e-10 floor of quantize.rs:39)
 *   q   = quantize_tensor(row, f64(s_r), 0, Int8) as i8   (quantize.rs:8-19) */
void tqo_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q, float* s) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * k;
        const double sc = fmax(absmax_of(row, k) / 127.0, 1e-10);
        const float sf = (float)sc;
        s[r] = sf;
        for (int64_t i = 0; i < k; ++i) {
            const double qd = rust_clamp(round((double)row[i] / (double)sf + 0.0), -128.0, 127.0);
            q[r * k + i] = (int8_t)rust_as_int(qd, -128.0, 127.0);
        }
    }
}

/* dequantize_tensor (quantize.rs:22-27) with zp = 0, result stored as f32 */
void tqo_dequantize_i8_rowwise(const int8_t* q, const float* s, int64_t rows, int64_t k,
                               float* w_hat) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < k; ++i)
            w_hat[r * k + i] = (float)(((double)q[r * k + i] - 0.0) * (double)s[r]);
}

/* Build-defined symmetric INT4, groups of 128 along K:
 *   s = max(f16_rne(absmax_g / 7), 2^-24)   (2^-24 = smallest positive f16; the
 *       f16 counterpart of the reference's 1e-10 floor, which f16 flushes to 0)
 *   q = quantize_tensor(group, f64(s), 0, Int4) as i8 in [-8, 7]
 *   byte[r, j] = (q[r, 2j] & 0xF) | (q[r, 2j+1] & 0xF) << 4   (low nibble = even k) */
void tqo_quantize_i4_g128(const float* w, int64_t rows, int64_t k, uint8_t* packed,
                          uint16_t* s_f16) {
    const int64_t groups = k / 128;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < groups; ++g) {
            const float* grp = w + r * k + g * 128;
            uint16_t h = tqo_f64_to_f16_bits(absmax_of(grp, 128) / 7.0);
            if (h == 0) h = 1;
            s_f16[r * groups + g] = h;
            const double sv = tqo_f16_bits_to_f64(h);
            for (int i = 0; i < 128; i += 2) {
                const double q0 = rust_clamp(round((double)grp[i] / sv + 0.0), -8.0, 7.0);
                const double q1 = rust_clamp(round((double)grp[i + 1] / sv + 0.0), -8.0, 7.0);
                const int c0 = rust_as_int(q0, -8.0, 7.0), c1 = rust_as_int(q1, -8.0, 7.0);
                packed[r * (k / 2) + g * 64 + i / 2] = (uint8_t)((c0 & 0xF) | ((c1 & 0xF) << 4));
            }
        }
}

static int nibble_value(uint8_t byte, int hi) {
    const int v = hi ? (byte >> 4) : (byte & 0xF);
    return v >= 8 ? v - 16 : v;
}

void tqo_dequantize_i4_g128(const uint8_t* packed, const uint16_t* s_f16, int64_t rows,
                            int64_t k, float* w_hat) {
    const int64_t groups = k / 128;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < k; ++i) {
            const int q = nibble_value(packed[r * (k / 2) + i / 2], (int)(i & 1));
            const double sv = tqo_f16_bits_to_f64(s_f16[r * groups + i / 128]);
            w_hat[r * k + i] = (float)(((double)q - 0.0) * sv);
        }
}

/* dequantized weight in f64, as Linear::from_tensors receives it (linear.rs:65-75) */
static double* deq_w8_f64(const int8_t* q, const float* s, int64_t n, int64_t k) {
    double* w = (double*)malloc(sizeof(double) * (size_t)(n * k));
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) w[r * k + i] = ((double)q[r * k + i] - 0.0) * (double)s[r];
    return w;
}

static double* deq_w4_f64(const uint8_t* packed, const uint16_t* s_f16, int64_t n, int64_t k) {
    double* w = (double*)malloc(sizeof(double) * (size_t)(n * k));
    const int64_t groups = k / 128;
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) {
            const int q = nibble_value(packed[r * (k / 2) + i / 2], (int)(i & 1));
            w[r * k + i] = ((double)q - 0.0) * tqo_f16_bits_to_f64(s_f16[r * groups + i / 128]);
        }
    return w;
}

void tqo_linear_w8(const float* x, int64_t m, const int8_t* q, const float* s,
                   const float* bias, int64_t n, int64_t k, double* y) {
    double* xd = (double*)malloc(sizeof(double) * (size_t)(m * k));
    for (int64_t i = 0; i < m * k; ++i) xd[i] = (double)x[i];
    double* w = deq_w8_f64(q, s, n, k);
    tqo_linear(xd, m, w, bias, n, k, y);
    free(w);
    free(xd);
}

void tqo_linear_w4g128_bf16(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                            const uint16_t* s_f16, const float* bias, int64_t n, int64_t k,
                            double* y) {
    double* xd = (double*)malloc(sizeof(double) * (size_t)(m * k));
    for (int64_t i = 0; i < m * k; ++i) xd[i] = tqo_bf16_bits_to_f64(x_bf16[i]);
    double* w = deq_w4_f64(packed, s_f16, n, k);
    tqo_linear(xd, m, w, bias, n, k, y);
    free(w);
    free(xd);
}

void tqo_linear_w4g128_f32(const float* x, int64_t m, const uint8_t* packed,
                           const uint16_t* s_f16, const float* bias, int64_t n, int64_t k,
                           double* y) {
    double* xd = (double*)malloc(sizeof(double) * (size_t)(m * k));
    for (int64_t i = 0; i < m * k; ++i) xd[i] = (double)x[i];
    double* w = deq_w4_f64(packed, s_f16, n, k);
    tqo_linear(xd, m, w, bias, n, k, y);
    free(w);
    free(xd);
}

/* Build-defined W8A8 accumulators: Tensor::mm over integral f64 codes is exact
 * (|acc| <= K*128*128 < 2^53), so the int32 result is the exact integer sum. */
void tqo_gemm_w8a8_acc(const int8_t* qa, const int8_t* qw, int64_t m, int64_t n, int64_t k,
                       int32_t* acc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            int64_t t = 0;
            for (int64_t p = 0; p < k; ++p) t += (int64_t)qa[i * k + p] * (int64_t)qw[j * k + p];
            acc[i * n + j] = (int32_t)t;
        }
}

/* Reference value of the W8A8 product: mm(deq(qa), deq(qw)^T) (+ b) in f64. */
void tqo_linear_w8a8(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                     const float* bias, int64_t m, int64_t n, int64_t k, double* y) {
    double* a = deq_w8_f64(qa, sa, m, k);
    double* w = deq_w8_f64(qw, sw, n, k);
    tqo_linear(a, m, w, bias, n, k, y);
    free(w);
    free(a);
}

/* Build-defined quantized FFN composed from Linear (linear.rs:111-121), SiLU
 * (activation.rs:70-74) and Tensor::mul (tensor_ops.rs:155-157), all in f64:
 *   h = SiLU(x Wg^T) * (x Wu^T);  y = h Wd^T */
void tqo_mlp_w4g128(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                    const uint8_t* pg, const uint16_t* sg, const uint8_t* pu,
                    const uint16_t* su, const uint8_t* pd, const uint16_t* sd, double* y) {
    double* g = (double*)malloc(sizeof(double) * (size_t)(m * f));
    double* u = (double*)malloc(sizeof(double) * (size_t)(m * f));
    tqo_linear_w4g128_bf16(x_bf16, m, pg, sg, NULL, f, d, g);
    tqo_linear_w4g128_bf16(x_bf16, m, pu, su, NULL, f, d, u);
    for (int64_t i = 0; i < m * f; ++i) g[i] = tqo_silu_module(g[i]) * u[i];
    free(u);
    double* w = deq_w4_f64(pd, sd, d, f);
    tqo_linear(g, m, w, NULL, d, f, y);
    free(w);
    free(g);
}

/* ---- build-defined FP8: OCP 8-bit float E4M3 ("e4m3fn") ----
 * Bits S.EEEE.MMM, exponent bias 7, no infinities, S.1111.111 = NaN.
 * Normal (E >= 1): (1 + M/8) * 2^(E-7); subnormal (E == 0): M * 2^-9.
 * Largest finite value 448 = 0x7E, the range of QuantDType::FP8
 * (crates/theano-quantize/src/qconfig.rs:29,38). */
double tqo_e4m3_to_f64(uint8_t b) {
    const double sign = (b & 0x80u) ? -1.0 : 1.0;
    const int e = (b >> 3) & 0xF;
    const int m = b & 7;
    if (e == 15 && m == 7) return NAN;
    if (e == 0) return sign * ldexp((double)m, -9);
    return sign * ldexp((double)(8 + m), e - 10);
}

/* Round to nearest, ties to even, on the e4m3 grid extended past 448 by one
 * step (480); a result of 480 or more, an infinity or a NaN encodes NaN with
 * the input's sign.  So 464 (the tie between 448 and 480) gives 448 and
 * anything above 464 gives NaN. */
uint8_t tqo_f32_to_e4m3(float x) {
    const uint8_t sign = signbit(x) ? 0x80u : 0u;
    if (x != x || isinf(x)) return (uint8_t)(sign | 0x7Fu);
    const double a = fabs((double)x);
    if (a < 0x1p-6) { /* subnormal range, ulp 2^-9; m == 8 is the smallest normal 0x08 */
        const double m = nearbyint(a * 0x1p9);
        return (uint8_t)(sign | (uint8_t)m);
    }
    int e2;
    frexp(a, &e2);
    int e = e2 - 1; /* a in [2^e, 2^(e+1)) */
    double m = nearbyint(ldexp(a, 3 - e)); /* in [8, 16] */
    if (m == 16.0) {
        m = 8.0;
        e += 1;
    }
    if (e + 7 > 15) return (uint8_t)(sign | 0x7Fu);
    return (uint8_t)(sign | (uint8_t)((e + 7) << 3) | (uint8_t)(m - 8.0)); /* e = 8, m = 15: 0x7F NaN */
}

/* Build-defined symmetric per-row FP8 (dynamic per-token for activations):
 *   s_r = f32(max(absmax_r / 448, 1e-10))     (qmax of QuantDType::FP8, the
 *                                              1e-10 floor of quantize.rs:39)
 *   q   = e4m3(clamp(f32(x / s_r), -448, 448)), NaN -> 0x7F
 * x / s_r is the correctly rounded f32 quotient (the f64 quotient rounded to
 * f32 is that: 53 >= 2 * 24 + 2), and the clamp keeps NaN (f64::clamp). */
void tqo_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q, float* s) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = w + r * k;
        const float sf = (float)fmax(absmax_of(row, k) / 448.0, 1e-10);
        s[r] = sf;
        for (int64_t i = 0; i < k; ++i) {
            const float v = (float)((double)row[i] / (double)sf);
            q[r * k + i] = v != v ? 0x7Fu : tqo_f32_to_e4m3((float)rust_clamp(v, -448.0, 448.0));
        }
    }
}

/* w_hat = f32(e4m3(q) * s[row]) (the f64 product of a 4-bit and a 24-bit
 * significand is exact, so this is one f32 rounding) */
void tqo_dequantize_fp8_rowwise(const uint8_t* q, const float* s, int64_t rows, int64_t k,
                                float* w_hat) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t i = 0; i < k; ++i)
            w_hat[r * k + i] = (float)(tqo_e4m3_to_f64(q[r * k + i]) * (double)s[r]);
}

static double* deq_fp8_f64(const uint8_t* q, const float* s, int64_t n, int64_t k) {
    double* w = (double*)malloc(sizeof(double) * (size_t)(n * k));
    for (int64_t r = 0; r < n; ++r)
        for (int64_t i = 0; i < k; ++i) w[r * k + i] = tqo_e4m3_to_f64(q[r * k + i]) * (double)s[r];
    return w;
}

/* Reference value of the FP8 W8A8 product: mm(deq(qa), deq(qw)^T) (+ b) in f64
 * (tensor_ops.rs:379-410, linear.rs:111-121). */
void tqo_linear_fp8(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                    const float* bias, int64_t m, int64_t n, int64_t k, double* y) {
    double* a = deq_fp8_f64(qa, sa, m, k);
    double* w = deq_fp8_f64(qw, sw, n, k);
    tqo_linear(a, m, w, bias, n, k, y);
    free(w);
    free(a);
}

/* ---- element type conversion (build-defined; the reference keeps f64 values
 * and a DType, crates/theano-types/src/dtype.rs:5-25, tensor.rs:277-299) ----
 * Type codes follow DType's order: F16 BF16 F32 F64 U8 I8 I16 I32 I64 Bool. */
uint16_t tqo_f64_to_bf16_bits(double x) {
    const uint16_t sign = signbit(x) ? 0x8000u : 0u;
    if (x != x) return (uint16_t)(sign | 0x7FC0u);
    const double a = fabs(x);
    /* largest finite bf16 is (2 - 2^-7) 2^127; half an ulp above rounds to inf */
    if (a >= ldexp(2.0 - ldexp(1.0, -8), 127)) return (uint16_t)(sign | 0x7F80u);
    if (a < 0x1p-126) { /* subnormal range, ulp 2^-133 */
        const double m = nearbyint(ldexp(a, 133));
        return (uint16_t)(sign | (uint16_t)m); /* m == 128 encodes 2^-126 */
    }
    int e2;
    frexp(a, &e2);
    int e = e2 - 1;
    double m = nearbyint(ldexp(a, 7 - e));
    if (m == 256.0) {
        m = 128.0;
        e += 1;
    }
    return (uint16_t)(sign | (uint16_t)((e + 127) << 7) | (uint16_t)(m - 128.0));
}

int64_t tqo_dtype_size(int t) {
    static const int64_t sz[10] = {2, 2, 4, 8, 1, 1, 2, 4, 8, 1};
    return (t >= 0 && t < 10) ? sz[t] : 0;
}

static double conv_get(const void* p, int t, int64_t i) {
    switch (t) {
        case 0: return tqo_f16_bits_to_f64(((const uint16_t*)p)[i]);
        case 1: return tqo_bf16_bits_to_f64(((const uint16_t*)p)[i]);
        case 2: return (double)((const float*)p)[i];
        case 3: return ((const double*)p)[i];
        case 4: return (double)((const uint8_t*)p)[i];
        case 5: return (double)((const int8_t*)p)[i];
        case 6: return (double)((const int16_t*)p)[i];
        case 7: return (double)((const int32_t*)p)[i];
        case 8: return (double)((const int64_t*)p)[i];
        default: return ((const uint8_t*)p)[i] ? 1.0 : 0.0;
    }
}

/* Rust `f64 as T` for an integer T with range [lo, hi]: toward zero,
 * saturating, NaN -> 0 */
static double rust_as(double x, double lo, double hi) {
    if (x != x) return 0.0;
    if (x <= lo) return lo;
    if (x >= hi) return hi;
    return trunc(x);
}

static void conv_put(void* p, int t, int64_t i, double v) {
    switch (t) {
        case 0: ((uint16_t*)p)[i] = tqo_f64_to_f16_bits(v); break;
        case 1: ((uint16_t*)p)[i] = tqo_f64_to_bf16_bits(v); break;
        case 2: ((float*)p)[i] = (float)v; break; /* C double -> float: IEEE RNE */
        case 3: ((double*)p)[i] = v; break;
        case 4: ((uint8_t*)p)[i] = (uint8_t)rust_as(v, 0.0, 255.0); break;
        case 5: ((int8_t*)p)[i] = (int8_t)rust_as(v, -128.0, 127.0); break;
        case 6: ((int16_t*)p)[i] = (int16_t)rust_as(v, -32768.0, 32767.0); break;
        case 7: ((int32_t*)p)[i] = (int32_t)rust_as(v, -2147483648.0, 2147483647.0); break;
        case 8: {
            /* 2^63 is not an i64; every double below it truncates exactly */
            if (v != v) ((int64_t*)p)[i] = 0;
            else if (v >= 0x1p63) ((int64_t*)p)[i] = INT64_MAX;
            else if (v <= -0x1p63) ((int64_t*)p)[i] = INT64_MIN;
            else ((int64_t*)p)[i] = (int64_t)trunc(v);
            break;
        }
        default: ((uint8_t*)p)[i] = (v != 0.0) ? 1u : 0u; break; /* NaN != 0 */
    }
}

void tqo_convert(const void* src, int src_t, void* dst, int dst_t, int64_t n) {
    for (int64_t i = 0; i < n; ++i) conv_put(dst, dst_t, i, conv_get(src, src_t, i));
}

/* ---- attention core of MultiheadAttention::forward_with_mask
 * (crates/theano-nn/src/transformer.rs:95-142), f64:
 *   scores = (q_h . k_h^T) * (1 / sqrt(D))  (+ mask[b or 0][i][j])
 *   P = softmax(scores) per row (tensor_ops.rs:574-620: max with f64::max,
 *       exp(x - max), sequential sum, divide), O_h = P . v_h.
 * q, k, v, out: [B*S, E] row-major, head h in columns [h*D, (h+1)*D), E = H*D.
 * mask: NULL or [mask_batch, S, S] (mask_batch 1 broadcasts over the batch). */
void tqo_attention(const double* q, const double* k, const double* v, const double* mask,
                   int64_t mask_batch, int64_t B, int64_t S, int64_t H, int64_t D, double* out) {
    const int64_t E = H * D;
    const double inv_scale = 1.0 / sqrt((double)D);
    double* row = (double*)malloc(sizeof(double) * (size_t)S);
    for (int64_t b = 0; b < B; ++b)
        for (int64_t h = 0; h < H; ++h)
            for (int64_t i = 0; i < S; ++i) {
                const double* qi = q + (b * S + i) * E + h * D;
                double mx = -INFINITY;
                for (int64_t j = 0; j < S; ++j) {
                    const double* kj = k + (b * S + j) * E + h * D;
                    double dot = 0.0;
                    for (int64_t d = 0; d < D; ++d) dot += qi[d] * kj[d];
                    double sc = dot * inv_scale;
                    if (mask) sc += mask[((mask_batch == 1 ? 0 : b) * S + i) * S + j];
                    row[j] = sc;
                    mx = fmax(mx, sc);
                }
                double sum = 0.0;
                for (int64_t j = 0; j < S; ++j) {
                    row[j] = exp(row[j] - mx);
                    sum += row[j];
                }
                for (int64_t j = 0; j < S; ++j) row[j] /= sum;
                double* oi = out + (b * S + i) * E + h * D;
                for (int64_t d = 0; d < D; ++d) {
                    double acc = 0.0;
                    for (int64_t j = 0; j < S; ++j) acc += row[j] * v[(b * S + j) * E + h * D + d];
                    oi[d] = acc;
                }
            }
    free(row);
}
