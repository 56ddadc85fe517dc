/* Checks the f32 arithmetic of the quantize coders against what it replaces:
 *   - rhaz_div (tq_internal.h) and code_i8_row (tq_rowfmt.h): a candidate biased
 *     2^-12 below the half-way points and one residual correction, against round
 *     half away from zero of the f64 quotient with the clamp (quantize.rs:8-19);
 *   - FmtFp8::Row::quot (tq_rowfmt.h): x * (1/s) with one fma correction, against
 *     IEEE x / s wherever either is >= 2^-12 (below that both code to a zero of
 *     x's sign in e4m3).
 * The same expressions as the device functions, compiled for the host with
 * -ffp-contract=off so every fmaf is one rounding.  Prints one line per check
 * and exits non-zero on any mismatch.  `bias` (argv[1], default 2^-12) lets a
 * caller show that a smaller bias fails. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float fbits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

static uint64_t rs = 0x9E3779B97F4A7C15ull;
static uint64_t rnd(void) { rs ^= rs << 13; rs ^= rs >> 7; rs ^= rs << 17; return rs; }
static float urand(void) { return (float)((rnd() >> 40) * 0x1p-24); }

static float bias = 0x1p-12f;

/* rhaz_div with NaN -> 0 */
static float rhaz_div(float a, float s, float inv, float half, float cap) {
    const float n = floorf(fminf(fmaxf(fmaf(a, inv, 0.5f - bias), 0.0f), cap));
    const float r = fmaf(-n, s, a);
    return (r >= half) ? n + 1.0f : n;
}
static int signed_code(float x, float n, int qmin, int qmax) {
    const int c = (int)copysignf(n, x);
    return c < qmin ? qmin : (c > qmax ? qmax : c);
}
static int code_i8_row(float x, float s, float inv, float half) {
    const float a = fabsf(x);
    float n = floorf(fmaxf(fmaf(a, inv, 0.5f - bias), 0.0f));
    const float r = fmaf(-n, s, a);
    n = (r >= half) ? n + 1.0f : n;
    return (int)copysignf(n, x);
}
/* round half away from zero of the f64 quotient, clamped; NaN -> 0 */
static int ref_code(float x, float s, int qmin, int qmax) {
    if (x != x) return 0;
    const double q = (double)x / (double)s;
    double n = q >= 0 ? floor(q + 0.5) : -floor(-q + 0.5);
    if (n > qmax) n = qmax;
    if (n < qmin) n = qmin;
    return (int)n;
}
static float scale_i8(float absmax) {
    const double d = (double)absmax / 127.0;
    return (float)(d > 1e-10 ? d : 1e-10);
}
static float scale_i4(float absmax) {
    const float h = (float)(_Float16)(float)((double)absmax / 7.0);
    return h == 0.0f ? 0x1p-24f : h;
}

/* x near (k + 1/2) s, d ulp away (d in [-3, 3]), random sign */
static float near_tie(float s, int kmax) {
    const int k = (int)(rnd() % (uint64_t)kmax);
    uint32_t b = bits((float)((k + 0.5) * (double)s));
    b += (int)(rnd() % 7) - 3;
    const float t = fbits(b);
    return (rnd() & 1) ? -t : t;
}

static long check_int(void) {
    long bad = 0, n = 0;
    for (int row = 0; row < 20000; ++row) {
        const float am = ldexpf(1.0f + urand(), (int)(rnd() % 160) - 140);
        const float s8 = scale_i8(am), s4 = scale_i4(am);
        for (int i = 0; i < 32; ++i) {
            const int kind = (int)(rnd() % 4);
            float x = kind == 0 ? (2 * urand() - 1) * am
                    : kind == 1 ? near_tie(s4, 40)
                    : kind == 2 ? near_tie(s8, 130)
                                : ((rnd() & 1) ? am : -am);
            if (fabsf(x) > am) x = copysignf(am, x);
            if (s4 < INFINITY) { /* the kernels code an infinite scale as zeros */
                ++n;
                if (signed_code(x, rhaz_div(fabsf(x), s4, 1.0f / s4, 0.5f * s4, 32.0f), -8, 7) !=
                    ref_code(x, s4, -8, 7))
                    ++bad;
            }
            ++n;
            if (signed_code(x, rhaz_div(fabsf(x), s8, 1.0f / s8, 0.5f * s8, 256.0f), -128, 127) !=
                ref_code(x, s8, -128, 127))
                ++bad;
            ++n;
            if (code_i8_row(x, s8, 1.0f / s8, 0.5f * s8) != ref_code(x, s8, -128, 127)) ++bad;
        }
    }
    const float sp[] = {0.0f, -0.0f, NAN, 0x1p-149f, -0x1p-149f};
    for (int i = 0; i < 5; ++i) {
        const float s = scale_i8(1.27e-8f);
        n += 2;
        if (code_i8_row(sp[i], s, 1.0f / s, 0.5f * s) != ref_code(sp[i], s, -128, 127)) ++bad;
        if (signed_code(sp[i], rhaz_div(fabsf(sp[i]), 0x1p-24f, 0x1p24f, 0x1p-25f, 32.0f), -8, 7) !=
            ref_code(sp[i], 0x1p-24f, -8, 7))
            ++bad;
    }
    printf("integer codes: %ld checked, %ld differ from the f64 rounding\n", n, bad);
    return bad;
}

static long check_fp8(void) {
    /* random scales, the 1e-10 floor, 1, 2 and all-ones mantissas */
    uint32_t sc[12] = {0x2edbe6ffu, 0x3f800000u, 0x40000000u, 0x3f7fffffu, 0x3effffffu, 0x3f800001u};
    for (int i = 6; i < 12; ++i) sc[i] = (uint32_t)(127 + (int)(rnd() % 56) - 33) << 23 | (uint32_t)(rnd() & 0x7fffff);
    long bad = 0, n = 0;
    for (int i = 0; i < 12; ++i) {
        const float s = fbits(sc[i]), inv = 1.0f / s;
        const uint32_t top = bits(449.0f * s);
        for (uint64_t u = rnd() % 509; u <= top; u += 509) { /* every 509th f32 in [0, 449 s] */
            const float x = fbits((uint32_t)u);
            const float d = x / s, q = x * inv;
            const float m = copysignf(fmaf(fmaf(-q, s, x), inv, q), x);
            ++n;
            if (bits(d) != bits(m) && (d >= 0x1p-12f || m >= 0x1p-12f)) ++bad;
            if (bits(-d) != bits(copysignf(fmaf(fmaf(q, s, -x), inv, -q), -x)) && (d >= 0x1p-12f || m >= 0x1p-12f))
                ++bad;
        }
    }
    printf("fp8 quotients: %ld checked, %ld differ from IEEE x / s at or above 2^-12\n", n, bad);
    return bad;
}

int main(int argc, char** argv) {
    if (argc > 1) bias = strtof(argv[1], NULL);
    const long bad = check_int() + (argc > 1 ? 0 : check_fp8());
    return bad != 0;
}
