// tq_decode_w4.hip -- decode-shaped INT4 group-128 quantized Linear on gfx950:
//   y[m, n] = sum_g s[n, g] * sum_{k in g} x[m, k] * q[n, k]  (+ b[n]),  M <= 16,
// the reference's Linear::forward (crates/theano-nn/src/linear.rs:111-121) over
// the dequantized weight (crates/theano-quantize/src/quantize.rs:22-27).
//
// HBM-bound weight stream on the matrix cores.  A block owns 16 output rows and
// its 8 waves split K into contiguous runs of kGPW groups.  Lane l (row l%16,
// quarter q = l/16) streams 16 bytes of its row per group (the 32 nibbles
// k = 128g + 32q .. +32); packed dword t of that slice is the MFMA B operand of
// k-step t, so one wave-wide load feeds four v_mfma_f32_16x16x32_bf16 (x tokens
// are the A rows, weight rows the B columns).  Only bit operations touch the
// nibbles: after xor 0x8 a nibble is q+8 and (q+8) | 0x4300 is the bf16 of
// 136+q, so the MFMA sums (136+q)*x and the kernel subtracts 136*sum(x) of the
// group before applying its f16 scale.
//
// Each wave stages the x slice of its own groups in a private LDS strip (same
// slot order as the unpacked nibbles, 136*group sums alongside), so no block
// barrier sits between the first weight bytes and the arithmetic.  Weight loads
// are unconditional (clamped addresses) and run kWin groups ahead; with the
// group loop unrolled at compile time every vmcnt wait is exact.  The 8 waves'
// partial sums meet in LDS in a fixed order.
#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kRowsPerBlock = 16;
constexpr int kWaves = 8;
constexpr int kBlock = 64 * kWaves;
constexpr int kMaxGPW = 16;  // K <= 16 * 8 * 128 = 16384
constexpr int kWin = 3;

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Packed dword of 8 nibbles (k .. k+7, two's complement) -> bf16 of 136+q in the
// slot order (k, k+2), (k+1, k+3), (k+4, k+6), (k+5, k+7).
__device__ __forceinline__ u32x4 unpack_w4(uint32_t w) {
    const uint32_t lo = (w ^ 0x88888888u) & 0x0F0F0F0Fu;         // q+8 of k, k+2, k+4, k+6
    const uint32_t hi = ((w >> 4) ^ 0x08888888u) & 0x0F0F0F0Fu;  // q+8 of k+1, k+3, k+5, k+7
    return u32x4{__builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u),
                 __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u),
                 __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u),
                 __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u)};
}

// 8 bf16 (x0,x1)(x2,x3)(x4,x5)(x6,x7) -> the same slot order (x0,x2)(x1,x3)(x4,x6)(x5,x7)
__device__ __forceinline__ u32x4 slot_order(u32x4 v) {
    return u32x4{(v.x & 0xFFFFu) | (v.y << 16), (v.x >> 16) | (v.y & 0xFFFF0000u),
                 (v.z & 0xFFFFu) | (v.w << 16), (v.z >> 16) | (v.w & 0xFFFF0000u)};
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Per-wave LDS strip: x [m tokens][kGPW * 16 8-blocks][16 B] (token stride padded
// by 16 B), then 136*group sums [kGPW][16 tokens] f32.  After the strips the
// block keeps its partial sums [kWaves][16 rows][16 tokens] f32.
__host__ __device__ constexpr int strip_token_stride(int gpw) { return gpw * 256 + 16; }
__host__ __device__ constexpr int strip_bytes(int m, int gpw) { return m * strip_token_stride(gpw) + gpw * 64; }
inline size_t lds_bytes(int m, int gpw) {
    return static_cast<size_t>(kWaves) * strip_bytes(m, gpw) + kWaves * 256 * 4;
}

template <int kGPW>
__global__ __launch_bounds__(kBlock) void k_decode_w4g128(const uint16_t* __restrict__ x, int m,
                                                          const uint8_t* __restrict__ packed,
                                                          const uint16_t* __restrict__ s16,
                                                          const float* __restrict__ bias, int64_t n,
                                                          int64_t k, float* __restrict__ y) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr int kTStride = strip_token_stride(kGPW);
    const int64_t G = k >> 7;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int sb = strip_bytes(m, kGPW);
    uint8_t* strip_x = lds + wave * sb;
    float* strip_sum = reinterpret_cast<float*>(strip_x + m * kTStride);
    float* part = reinterpret_cast<float*>(lds + kWaves * sb);

    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + r16;
    const int64_t rowc = row < n ? row : n - 1;  // rows past n re-read row n-1; never stored
    const int64_t g0 = min<int64_t>(G, static_cast<int64_t>(wave) * kGPW);
    const int ng = static_cast<int>(min<int64_t>(G, g0 + kGPW) - g0);  // < kGPW only for trailing waves
    // slots past this wave's range re-read its last group; their results are masked
    const int64_t glast = max<int64_t>(0, min(G - 1, g0 + ng - 1));
    const uint8_t* wrow = packed + rowc * (k >> 1) + 16 * q;
    const uint16_t* srow = s16 + rowc * G;

    // This wave's x slice: 8-block b (of kGPW*16) of token t, 16 lanes per group.
    // The first items are loaded before the weights (vmcnt completes in order:
    // staging them then waits for x alone), any further ones (many tokens) after.
    const int items = m * kGPW * 16;
    auto x_at = [&](int idx) {
        const int t = idx / (kGPW * 16), b = idx - t * (kGPW * 16);
        const int64_t gk = min<int64_t>(g0 * 16 + b, G * 16 - 1);  // clamp for trailing waves
        return *reinterpret_cast<const u32x4*>(x + t * k + gk * 8);
    };
    auto stage = [&](int idx, const u32x4& v) {
        const int t = idx / (kGPW * 16), b = idx - t * (kGPW * 16);
        *reinterpret_cast<u32x4*>(strip_x + t * kTStride + b * 16) = slot_order(v);
        float sum = bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y) + bf16_lo(v.z) + bf16_hi(v.z) +
                    bf16_lo(v.w) + bf16_hi(v.w);
        sum = lane_group_sum<16>(sum);  // a group's 16 lanes (one DPP row) are all active
        if ((b & 15) == 0) strip_sum[(b >> 4) * 16 + t] = 136.0f * sum;
    };
    constexpr int kPre = 4 * kGPW < 8 ? 4 * kGPW : 8;  // items per lane loaded up front
    u32x4 xp[kPre];
#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int idx = lane + i * kWave;
        xp[i] = idx < items ? x_at(idx) : u32x4{0u, 0u, 0u, 0u};
    }

    // first window of weight and scale loads
    u32x4 wq[kWin];
    uint16_t sq[kWin];
#pragma unroll
    for (int i = 0; i < kWin && i < kGPW; ++i) {
        const int64_t g = min(g0 + i, glast);
        wq[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + g * 64));
        sq[i] = srow[g];
    }

#pragma unroll
    for (int i = 0; i < kPre; ++i) {
        const int idx = lane + i * kWave;
        if (idx < items) stage(idx, xp[i]);
    }
    for (int idx = lane + kPre * kWave; idx < items; idx += kWave) stage(idx, x_at(idx));
    // the strip is private to this wave: LDS accesses of one wave complete in order

    // dummy token rows (>= m) read token m-1; their results are never stored
    const int tok = r16 < m ? r16 : m - 1;
    const uint8_t* xa = strip_x + tok * kTStride + 64 * q;
    const int tq4 = 4 * q < m ? 4 * q : 0;  // correction rows of dummy tokens are never stored
    f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int slot = i % kWin;
        const uint32_t words[4] = {wq[slot].x, wq[slot].y, wq[slot].z, wq[slot].w};
        u32x4 a[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] = *reinterpret_cast<const u32x4*>(xa + (i * 16 + j) * 16);
        f32x4 t = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) t = mfma_bf16(a[j], unpack_w4(words[j]), t);
        const float sc = (i < ng) ? __half2float(__ushort_as_half(sq[slot])) : 0.0f;
        const f32x4 xs = *reinterpret_cast<const f32x4*>(strip_sum + i * 16 + tq4);
        acc.x = fmaf(sc, t.x - xs.x, acc.x);
        acc.y = fmaf(sc, t.y - xs.y, acc.y);
        acc.z = fmaf(sc, t.z - xs.z, acc.z);
        acc.w = fmaf(sc, t.w - xs.w, acc.w);
        if (i + kWin < kGPW) {  // compile-time: refill this slot with the group kWin ahead
            const int64_t gn = min(g0 + i + kWin, glast);
            wq[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + gn * 64));
            sq[slot] = srow[gn];
        }
    }

    // lane holds D[token 4q + r][row r16]; the waves' partials meet in a fixed order
    *reinterpret_cast<f32x4*>(part + (wave * 16 + r16) * 16 + 4 * q) = acc;
    __syncthreads();
    for (int i = tid; i < m * kRowsPerBlock; i += kBlock) {
        const int t = i / kRowsPerBlock, r = i - t * kRowsPerBlock;
        const int64_t orow = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + r;
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += part[(w * 16 + r) * 16 + t];
        if (orow < n) y[t * n + orow] = s + (bias ? bias[orow] : 0.0f);
    }
}

template <int kGPW>
int launch_one(int64_t blocks, int m, hipStream_t st, const uint16_t* x, const uint8_t* p, const uint16_t* s,
               const float* b, int64_t n, int64_t k, float* y) {
    static std::atomic<uint64_t> lds_set{0};  // allow the full 160 KB of LDS per block, per device
    if (int rc = allow_dynamic_lds(reinterpret_cast<const void*>(k_decode_w4g128<kGPW>), 160 * 1024, lds_set))
        return rc;
    k_decode_w4g128<kGPW><<<static_cast<unsigned>(blocks), kBlock, lds_bytes(m, kGPW), st>>>(x, m, p, s, b, n, k, y);
    return TQ_OK;
}

template <int kGPW = 1>
int launch_decode(int gpw, int64_t blocks, int m, hipStream_t st, const uint16_t* x, const uint8_t* p,
                  const uint16_t* s, const float* b, int64_t n, int64_t k, float* y) {
    if constexpr (kGPW < kMaxGPW) {
        if (gpw > kGPW) return launch_decode<kGPW + 1>(gpw, blocks, m, st, x, p, s, b, n, k, y);
    }
    return launch_one<kGPW>(blocks, m, st, x, p, s, b, n, k, y);
}

}  // namespace
}  // namespace tq

using namespace tq;

// Decode-shaped INT4 g128 Linear; tokens beyond what one block's LDS holds run
// as several passes over the weights.
extern "C" int tq_gemv_w4g128(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                              const uint16_t* s_f16, const float* bias, int64_t n, int64_t k, float* y,
                              tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemv_w4g128: negative shape");
    TQ_REQUIRE(m <= 16, "tq_gemv_w4g128: M=%lld > 16 (use tq_gemm_w4g128_bf16)", (long long)m);
    TQ_REQUIRE(k % 128 == 0, "tq_gemv_w4g128: K=%lld is not a multiple of 128", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(y, "tq_gemv_w4g128: null y");
    TQ_REQUIRE(k == 0 || (x_bf16 && packed && s_f16), "tq_gemv_w4g128: null pointer");
    TQ_REQUIRE(aligned(x_bf16, 2) && aligned(s_f16, 2) && (!bias || aligned(bias, 4)) && aligned(y, 4),
               "tq_gemv_w4g128: misaligned pointer");
    const int64_t gpw = ((k >> 7) + kWaves - 1) / kWaves;
    // the MFMA kernel keeps the tokens' K in LDS and streams 16-byte weight vectors
    if (k == 0 || gpw > kMaxGPW || !aligned(x_bf16, 16) || !aligned(packed, 16))
        return launch_linear_w4_generic(x_bf16, m, packed, s_f16, bias, n, k, y, as_hip(stream));
    const int64_t blocks = (n + kRowsPerBlock - 1) / kRowsPerBlock;
    TQ_REQUIRE(blocks < (int64_t(1) << 31), "tq_gemv_w4g128: N too large");
    const size_t lds_cap = 160 * 1024;
    int per_pass = static_cast<int>(m);
    while (per_pass > 1 && lds_bytes(per_pass, static_cast<int>(gpw)) > lds_cap) --per_pass;
    const hipStream_t st = as_hip(stream);
    for (int64_t m0 = 0; m0 < m; m0 += per_pass) {
        const int mm = static_cast<int>((m - m0) < per_pass ? (m - m0) : per_pass);
        int rc = launch_decode(static_cast<int>(gpw), blocks, mm, st, x_bf16 + m0 * k, packed, s_f16, bias, n, k,
                               y + m0 * n);
        if (rc == TQ_OK) rc = check_launch("tq_gemv_w4g128");
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}
