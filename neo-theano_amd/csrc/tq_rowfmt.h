// tq_rowfmt.h -- per-row symmetric formats shared by the quantize kernels and
// the decode GEMVs that quantize their activations in place: the row scale,
// the INT8 and FP8 (OCP e4m3) coders and the code values.
#pragma once

#include "tq_internal.h"

namespace tq {

// Symmetric absmax from a NaN-ignoring fold of |x| started at -inf: a row with
// no non-NaN value folds to -inf, which the observer form
// max(|min|, |max|) with min=+inf, max=-inf turns into +inf.
__device__ __forceinline__ float absmax_finish(float m) { return (m == -INFINITY) ? INFINITY : m; }

// INT8 code of x for scale s (finite, > 0).
__device__ __forceinline__ int code_i8(float x, float s, float inv_s, float half_s) {
    const float n = rhaz_div(fabsf(x), s, inv_s, half_s, 256.0f);
    return signed_code(x, n, -128, 127);
}

// INT8 code of x for its row's own scale s = f32(max(absmax/127, 1e-10)) (finite),
// round half away from zero of |x| / s, exact: rhaz_div's one-sided rounding
// without its cap, since q = |x| / s <= 127 (1 + 2^-23) gives n <= 127 (the code
// is in [-127, 127], no clamp).  fmax(NaN, 0) = 0 sends NaN to code 0 (its
// residual is NaN: no correction).
__device__ __forceinline__ int code_i8_row(float x, float s, float inv_s, float half_s) {
    const float a = fabsf(x);
    float n = floorf(fmaxf(fmaf(a, inv_s, 0.5f - 0x1p-12f), 0.0f));
    const float r = fmaf(-n, s, a);
    n = (r >= half_s) ? n + 1.0f : n;
    return static_cast<int>(copysignf(n, x));
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    // low bytes of a, b (bytes 0, 1) and c, d (bytes 2, 3)
    return __builtin_amdgcn_perm(static_cast<uint32_t>(b), static_cast<uint32_t>(a), 0x0c0c0400u) |
           __builtin_amdgcn_perm(static_cast<uint32_t>(d), static_cast<uint32_t>(c), 0x04000c0cu);
}

// ---- per-row symmetric formats ----
// Each format gives its qmax (s = f32(max(absmax / qmax, 1e-10))), a per-row
// coder built from s, and the value of a code: value(code) * s is the
// dequantized element.

// INT8: code = clamp(rhaz(x / s), -128, 127), NaN -> 0; an infinite scale (a row
// holding an infinity) gives all-zero codes (|x| / inf = 0, inf / inf = NaN -> 0).
struct FmtI8 {
    typedef int8_t code_t;
    static constexpr double kQmax = 127.0;
    struct Row {
        float s, inv, half;
        bool finite;
        __device__ explicit Row(float sc) : s(sc), inv(1.0f / sc), half(0.5f * sc), finite(sc < INFINITY) {}
        __device__ uint32_t code4(f32x4 v) const {
            if (!finite) return 0u;
            return pack4_i8(code_i8_row(v.x, s, inv, half), code_i8_row(v.y, s, inv, half),
                            code_i8_row(v.z, s, inv, half), code_i8_row(v.w, s, inv, half));
        }
        __device__ code_t code1(float x) const { return static_cast<code_t>(finite ? code_i8(x, s, inv, half) : 0); }
    };
    __device__ static f32x4 value4(uint32_t c, float sc) {
        f32x4 o;
        o.x = static_cast<float>(static_cast<int8_t>(c & 0xFF)) * sc;
        o.y = static_cast<float>(static_cast<int8_t>((c >> 8) & 0xFF)) * sc;
        o.z = static_cast<float>(static_cast<int8_t>((c >> 16) & 0xFF)) * sc;
        o.w = static_cast<float>(static_cast<int8_t>((c >> 24) & 0xFF)) * sc;
        return o;
    }
    __device__ static float value1(code_t c, float sc) { return static_cast<float>(c) * sc; }
};

// FP8 (OCP e4m3: bias 7, largest finite 448, S.1111.111 = NaN):
// code = e4m3_rne(clamp(f32(x / s), -448, 448)), NaN -> 0x7F.  x / s is the
// correctly rounded quotient (FmtFp8::Row::quot); v_cvt_pk_fp8_f32 rounds to
// nearest even and, after the clamp, never overflows.
__device__ __forceinline__ float sat448(float t) { return fminf(fmaxf(t, -448.0f), 448.0f); }

__device__ __forceinline__ uint32_t pack4_e4m3(float t0, float t1, float t2, float t3) {
    uint32_t w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat448(t0), sat448(t1), 0, false));
    w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(sat448(t2), sat448(t3), static_cast<int>(w), true));
    const uint32_t nan = (t0 != t0 ? 0x000000FFu : 0u) | (t1 != t1 ? 0x0000FF00u : 0u) |
                         (t2 != t2 ? 0x00FF0000u : 0u) | (t3 != t3 ? 0xFF000000u : 0u);
    return (w & ~nan) | (0x7F7F7F7Fu & nan);
}

struct FmtFp8 {
    typedef uint8_t code_t;
    static constexpr double kQmax = 448.0;
    // x / s for the row's own finite scale by one correction of x * (1/s)
    // (Markstein: q = x * inv, r = fma(-q, s, x) exact, q + r * inv rounded once),
    // with x's sign.  Over every x in [0, 449 s] for 35 scales (random, 1e-10, 1,
    // 2, all-ones mantissas) it equals IEEE x / s wherever either is >= 2^-12;
    // below that the residual underflows, and both code to a zero of x's sign.
    // An infinite scale (a row holding an infinity) takes the division.
    struct Row {
        float s, inv;
        bool finite;
        __device__ explicit Row(float sc) : s(sc), inv(1.0f / sc), finite(sc < INFINITY) {}
        __device__ float quot(float x) const {
            const float q = x * inv;
            return copysignf(fmaf(fmaf(-q, s, x), inv, q), x);
        }
        __device__ uint32_t code4(f32x4 v) const {
            if (!finite) return pack4_e4m3(v.x / s, v.y / s, v.z / s, v.w / s);
            return pack4_e4m3(quot(v.x), quot(v.y), quot(v.z), quot(v.w));
        }
        __device__ code_t code1(float x) const {
            return static_cast<code_t>(pack4_e4m3(finite ? quot(x) : x / s, 0.f, 0.f, 0.f) & 0xFF);
        }
    };
    __device__ static f32x4 value4(uint32_t c, float sc) {
        const int ci = static_cast<int>(c);
        f32x4 o;
        o.x = __builtin_amdgcn_cvt_f32_fp8(ci, 0) * sc;
        o.y = __builtin_amdgcn_cvt_f32_fp8(ci, 1) * sc;
        o.z = __builtin_amdgcn_cvt_f32_fp8(ci, 2) * sc;
        o.w = __builtin_amdgcn_cvt_f32_fp8(ci, 3) * sc;
        return o;
    }
    __device__ static float value1(code_t c, float sc) { return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(c), 0) * sc; }
};

// s = f32(max(absmax / qmax, 1e-10)), division in f64 (correctly rounded).
template <class Fmt>
__device__ __forceinline__ float row_scale(float absmax) {
    return static_cast<float>(fmax(static_cast<double>(absmax) / Fmt::kQmax, 1e-10));
}

}  // namespace tq
