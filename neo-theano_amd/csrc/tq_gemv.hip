// tq_gemv.hip -- decode-shaped quantized Linear (y = x . dequant(W)^T + b)
// for gfx950, the reference's Linear::forward (crates/theano-nn/src/linear.rs:111-121)
// over the dequantized weight of quantize.rs:22-27.
//
// Both kernels are HBM-bound weight streams: a wave owns whole output rows,
// each lane streams 16-byte slices of the row with global_load_dwordx4, keeps
// its slice of x in registers for the life of the wave, and the row's partial
// dot products meet in one wave64 butterfly.  M (tokens) <= 4 per pass; larger
// M runs as several passes.
//
// INT4 g128: nibbles become bf16 in registers with two bit operations
// ((q+8) | 0x4300 is the bf16 of 136+q), v_dot2_f32_bf16 multiplies them by x
// pairs, and 136*sum(x) is taken off once per 32-element slice before the f16
// group scale is applied.
#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                           false);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

constexpr int kBlock = 256;
constexpr int kWaves = kBlock / kWave;

// --------------------------------------------------------------- INT4 g128
// Chunk c of a row covers k in [2048c, 2048c + 2048): lane l owns the 16 bytes
// (32 nibbles) at k = 2048c + 32l, i.e. one quarter of group 16c + l/4.
template <int kM, int kChunks, int kRows>
__global__ __launch_bounds__(kBlock) void k_gemv_w4g128(const uint16_t* __restrict__ x,
                                                        int64_t x_stride,
                                                        const uint8_t* __restrict__ packed,
                                                        const uint16_t* __restrict__ s16,
                                                        const float* __restrict__ bias, int64_t n,
                                                        int64_t k, float* __restrict__ y,
                                                        int64_t y_stride) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWaves;
    const int64_t row_bytes = k >> 1;
    const int64_t groups = k >> 7;

    // x slice of this lane in register pairs matching the nibble pairing
    // (k, k+4), (k+1, k+5), (k+2, k+6), (k+3, k+7) of every packed dword.
    uint32_t xp[kM][kChunks][16];
    float xs[kM][kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int64_t kb = 2048 * c + 32 * lane;
        const bool valid = kb < k;
#pragma unroll
        for (int m = 0; m < kM; ++m) {
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                u32x4 v = u32x4{0, 0, 0, 0};
                if (valid) v = *reinterpret_cast<const u32x4*>(x + m * x_stride + kb + 8 * j);
                xp[m][c][4 * j + 0] = (v.x & 0xFFFFu) | (v.z << 16);
                xp[m][c][4 * j + 1] = (v.x >> 16) | (v.z & 0xFFFF0000u);
                xp[m][c][4 * j + 2] = (v.y & 0xFFFFu) | (v.w << 16);
                xp[m][c][4 * j + 3] = (v.y >> 16) | (v.w & 0xFFFF0000u);
                sum += bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y) + bf16_lo(v.z) +
                       bf16_hi(v.z) + bf16_lo(v.w) + bf16_hi(v.w);
            }
            xs[m][c] = sum * 136.0f;
        }
    }

    for (int64_t row0 = wave * kRows; row0 < n; row0 += nwaves * kRows) {
        u32x4 wq[kRows][kChunks];
        float sc[kRows][kChunks];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int64_t row = row0 + r;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int64_t kb = 2048 * c + 32 * lane;
                if (row < n && kb < k) {
                    wq[r][c] = __builtin_nontemporal_load(
                        reinterpret_cast<const u32x4*>(packed + row * row_bytes + (kb >> 1)));
                    sc[r][c] = __half2float(__ushort_as_half(s16[row * groups + (kb >> 7)]));
                } else {
                    wq[r][c] = u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
                    sc[r][c] = 0.0f;
                }
            }
        }
        float acc[kRows][kM];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[r][m] = 0.0f;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const uint32_t words[4] = {wq[r][c].x, wq[r][c].y, wq[r][c].z, wq[r][c].w};
                float p[kM];
#pragma unroll
                for (int m = 0; m < kM; ++m) p[m] = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t w = words[j] ^ 0x88888888u;
                    const uint32_t a0 = (w & 0x000F000Fu) | 0x43004300u;
                    const uint32_t a1 = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
                    const uint32_t a2 = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
                    const uint32_t a3 = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
#pragma unroll
                    for (int m = 0; m < kM; ++m) {
                        p[m] = dot2_bf16(a0, xp[m][c][4 * j + 0], p[m]);
                        p[m] = dot2_bf16(a1, xp[m][c][4 * j + 1], p[m]);
                        p[m] = dot2_bf16(a2, xp[m][c][4 * j + 2], p[m]);
                        p[m] = dot2_bf16(a3, xp[m][c][4 * j + 3], p[m]);
                    }
                }
#pragma unroll
                for (int m = 0; m < kM; ++m) acc[r][m] = fmaf(sc[r][c], p[m] - xs[m][c], acc[r][m]);
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int64_t row = row0 + r;
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                const float v = wave_sum(acc[r][m]);
                if (lane == 0 && row < n) y[m * y_stride + row] = v + (bias ? bias[row] : 0.0f);
            }
        }
    }
}

// ------------------------------------------------------------------- INT8
// Chunk c covers k in [1024c, 1024c + 1024): lane l owns the 16 codes at
// k = 1024c + 16l.  y = s[row] * sum(q * x) + b.
template <int kM, int kChunks, int kRows>
__global__ __launch_bounds__(kBlock) void k_gemv_w8(const float* __restrict__ x, int64_t x_stride,
                                                    const int8_t* __restrict__ q,
                                                    const float* __restrict__ s,
                                                    const float* __restrict__ bias, int64_t n,
                                                    int64_t k, float* __restrict__ y,
                                                    int64_t y_stride) {
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t wave = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    const int64_t nwaves = static_cast<int64_t>(gridDim.x) * kWaves;

    float xr[kM][kChunks][16];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) {
        const int64_t kb = 1024 * c + 16 * lane;
        const bool valid = kb < k;
#pragma unroll
        for (int m = 0; m < kM; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
                if (valid) v = *reinterpret_cast<const f32x4*>(x + m * x_stride + kb + 4 * j);
                xr[m][c][4 * j + 0] = v.x;
                xr[m][c][4 * j + 1] = v.y;
                xr[m][c][4 * j + 2] = v.z;
                xr[m][c][4 * j + 3] = v.w;
            }
    }

    for (int64_t row0 = wave * kRows; row0 < n; row0 += nwaves * kRows) {
        i32x4 wq[kRows][kChunks];
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int64_t row = row0 + r;
                const int64_t kb = 1024 * c + 16 * lane;
                wq[r][c] = (row < n && kb < k)
                               ? __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(q + row * k + kb))
                               : i32x4{0, 0, 0, 0};
            }
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            float acc[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[m] = 0.0f;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int words[4] = {wq[r][c].x, wq[r][c].y, wq[r][c].z, wq[r][c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
#pragma unroll
                    for (int b = 0; b < 4; ++b) {
                        const float wv = static_cast<float>(static_cast<int8_t>((words[j] >> (8 * b)) & 0xFF));
#pragma unroll
                        for (int m = 0; m < kM; ++m) acc[m] = fmaf(wv, xr[m][c][4 * j + b], acc[m]);
                    }
            }
            const int64_t row = row0 + r;
            const float sc = row < n ? s[row] : 0.0f;
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                const float v = wave_sum(acc[m]);
                if (lane == 0 && row < n) y[m * y_stride + row] = sc * v + (bias ? bias[row] : 0.0f);
            }
        }
    }
}

template <int kM, int kChunks>
void launch_w4(const uint16_t* x, int64_t xs, const uint8_t* p, const uint16_t* s, const float* b,
               int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    constexpr int kRows = 2;
    const int64_t waves = (n + kRows - 1) / kRows;
    const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;  // 8 blocks = 32 waves per CU
    int64_t blocks = (waves + kWaves - 1) / kWaves;
    if (blocks > cap) blocks = cap;
    k_gemv_w4g128<kM, kChunks, kRows><<<static_cast<unsigned>(blocks), kBlock, 0, st>>>(x, xs, p, s, b, n, k,
                                                                                      y, ys);
}

template <int kM>
void dispatch_w4(int chunks, const uint16_t* x, int64_t xs, const uint8_t* p, const uint16_t* s,
                 const float* b, int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    switch (chunks) {
    case 1: launch_w4<kM, 1>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 2: launch_w4<kM, 2>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 3: launch_w4<kM, 3>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 4: launch_w4<kM, 4>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 5: launch_w4<kM, 5>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 6: launch_w4<kM, 6>(x, xs, p, s, b, n, k, y, ys, st); break;
    case 7: launch_w4<kM, 7>(x, xs, p, s, b, n, k, y, ys, st); break;
    default: launch_w4<kM, 8>(x, xs, p, s, b, n, k, y, ys, st); break;
    }
}

template <int kM, int kChunks>
void launch_w8(const float* x, int64_t xs, const int8_t* q, const float* s, const float* b,
               int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    constexpr int kRows = 2;
    const int64_t waves = (n + kRows - 1) / kRows;
    const int64_t cap = static_cast<int64_t>(device_cu_count()) * 8;
    int64_t blocks = (waves + kWaves - 1) / kWaves;
    if (blocks > cap) blocks = cap;
    k_gemv_w8<kM, kChunks, kRows><<<static_cast<unsigned>(blocks), kBlock, 0, st>>>(x, xs, q, s, b, n, k, y,
                                                                                  ys);
}

template <int kM>
void dispatch_w8(int chunks, const float* x, int64_t xs, const int8_t* q, const float* s,
                 const float* b, int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    switch (chunks) {
    case 1: launch_w8<kM, 1>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 2: launch_w8<kM, 2>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 3: launch_w8<kM, 3>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 4: launch_w8<kM, 4>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 5: launch_w8<kM, 5>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 6: launch_w8<kM, 6>(x, xs, q, s, b, n, k, y, ys, st); break;
    case 7: launch_w8<kM, 7>(x, xs, q, s, b, n, k, y, ys, st); break;
    default: launch_w8<kM, 8>(x, xs, q, s, b, n, k, y, ys, st); break;
    }
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_gemv_w4g128(const uint16_t* x_bf16, int64_t m, const uint8_t* packed, const uint16_t* s_f16,
                   const float* bias, int64_t n, int64_t k, float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemv_w4g128: negative shape");
    TQ_REQUIRE(m <= 16, "tq_gemv_w4g128: M=%lld > 16 (use tq_gemm_w4g128_bf16)", (long long)m);
    TQ_REQUIRE(k % 128 == 0, "tq_gemv_w4g128: K=%lld is not a multiple of 128", (long long)k);
    TQ_REQUIRE(k <= 8 * 2048, "tq_gemv_w4g128: K=%lld > 16384", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(y, "tq_gemv_w4g128: null y");
    if (k == 0) return fail(TQ_EINVAL, "tq_gemv_w4g128: K=0");
    TQ_REQUIRE(x_bf16 && packed && s_f16, "tq_gemv_w4g128: null pointer");
    TQ_REQUIRE(aligned(x_bf16, 16) && aligned(packed, 16) && aligned(s_f16, 2) &&
                   (!bias || aligned(bias, 4)) && aligned(y, 4),
               "tq_gemv_w4g128: misaligned pointer (x and packed need 16 B)");
    const int chunks = static_cast<int>((k + 2047) / 2048);
    const hipStream_t st = as_hip(stream);
    // passes of up to 4 tokens; tokens per pass limited so x fits in registers
    const int64_t per_pass = chunks <= 2 ? 4 : (chunks <= 4 ? 2 : 1);
    for (int64_t m0 = 0; m0 < m; m0 += per_pass) {
        const int64_t mm = (m - m0) < per_pass ? (m - m0) : per_pass;
        const uint16_t* xp = x_bf16 + m0 * k;
        float* yp = y + m0 * n;
        if (mm == 1) dispatch_w4<1>(chunks, xp, k, packed, s_f16, bias, n, k, yp, n, st);
        else if (mm == 2) dispatch_w4<2>(chunks, xp, k, packed, s_f16, bias, n, k, yp, n, st);
        else if (mm == 3) dispatch_w4<3>(chunks, xp, k, packed, s_f16, bias, n, k, yp, n, st);
        else dispatch_w4<4>(chunks, xp, k, packed, s_f16, bias, n, k, yp, n, st);
        const int rc = check_launch("tq_gemv_w4g128");
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

int tq_gemv_w8(const float* x, int64_t m, const int8_t* q, const float* s, const float* bias,
               int64_t n, int64_t k, float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemv_w8: negative shape");
    TQ_REQUIRE(m <= 16, "tq_gemv_w8: M=%lld > 16 (use tq_gemm_w8a8)", (long long)m);
    TQ_REQUIRE(k % 16 == 0, "tq_gemv_w8: K=%lld is not a multiple of 16", (long long)k);
    TQ_REQUIRE(k <= 8 * 1024, "tq_gemv_w8: K=%lld > 8192", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(y, "tq_gemv_w8: null y");
    if (k == 0) return fail(TQ_EINVAL, "tq_gemv_w8: K=0");
    TQ_REQUIRE(x && q && s, "tq_gemv_w8: null pointer");
    TQ_REQUIRE(aligned(x, 16) && aligned(q, 16) && aligned(s, 4) && (!bias || aligned(bias, 4)) &&
                   aligned(y, 4),
               "tq_gemv_w8: misaligned pointer (x and q need 16 B)");
    const int chunks = static_cast<int>((k + 1023) / 1024);
    const hipStream_t st = as_hip(stream);
    const int64_t per_pass = chunks <= 2 ? 4 : (chunks <= 4 ? 2 : 1);
    for (int64_t m0 = 0; m0 < m; m0 += per_pass) {
        const int64_t mm = (m - m0) < per_pass ? (m - m0) : per_pass;
        const float* xp = x + m0 * k;
        float* yp = y + m0 * n;
        if (mm == 1) dispatch_w8<1>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 2) dispatch_w8<2>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 3) dispatch_w8<3>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else dispatch_w8<4>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        const int rc = check_launch("tq_gemv_w8");
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

}  // extern "C"
