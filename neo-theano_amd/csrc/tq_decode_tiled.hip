// tq_decode_tiled.hip -- decode-shaped INT4 group-128 Linear on a row-tiled
// copy of the packed weight, for gfx950.  Same result as tq_gemv_w4g128 (the
// reference's Linear::forward over the dequantized weight,
// crates/theano-nn/src/linear.rs:111-121, quantize.rs:22-27); only the byte
// order of the weight differs.
//
// Tiled layout (a permutation of the canonical [N, K/2] bytes; T rows per tile,
// C = K/32 chunks of 16 bytes per row, G = K/128 groups, rows padded to a
// multiple of T with zero bytes and zero scales):
//   packed_t[((t*C + c)*T + r)*16 + b] = packed[t*T + r][16c + b]
//   s_t[(t*G + g)*T + r]               = s[t*T + r][g]
// so the 16-byte chunk c of the T rows of a tile is one contiguous T*16-byte run.
//
// Three kernels read this layout:
//  * k_decode_diag (1-4 tokens, T = 16, 32 or 64; the decode path): one block of
//    16 waves per tile, waves split K by groups.  Every packed dword of a lane is
//    the A operand of one v_mfma_f32_16x16x32_bf16; the 4 k-groups of the MFMA
//    are kR = T/16 row groups times 4/kR consecutive chunks, and the B operand
//    carries token j's x only in the k-groups of row group c % kR for column
//    c = j kR + (row group), zeros elsewhere, so the product's columns are the
//    (token, row group) dot products (details at the kernel).  The vector ALU
//    only unpacks nibbles (7 instructions per dword); x is staged once per wave
//    in LDS.
//    The same kernel runs the decode FFN: gate and up rows share 64-row tiles and
//    the block applies SiLU(g) * u, then the down projection takes h as bf16
//    hi + lo rows and adds the two halves per token.
//  * k_decode_tiled (fallback for other tile heights): one block (16 waves) per
//    tile, lane = row, waves split the chunks.
// x is wave-uniform, so each wave permutes its slice of x once into a private
// LDS strip and reads it back with broadcast ds_read_b128; no cross-lane
// reduction is needed per row.  Nibbles become bf16 with bit operations
// ((q+8) | 0x4300 is the bf16 of 136+q), v_dot2_f32_bf16 multiplies them by x
// pairs, 136*sum(x) of each 32-element chunk is subtracted before the f16
// group scale is applied.  Weight loads are unconditional (clamped addresses)
// and run kWin chunks ahead of the arithmetic; the waves' partial sums meet in
// LDS in a fixed order.  Its arithmetic grows with the token count.
//  * k_decode_tiled_mfma (5-16 tokens, T a multiple of 16): unpacked bf16
//    weights feed v_mfma_f32_16x16x32_bf16 with the tokens as the other operand,
//    so the cost is nearly flat in the token count.  Each wave owns the whole
//    tile and a run of groups, reads its tokens' x straight from L2 (no LDS
//    staging, no barrier before the arithmetic) and consumes its loads in
//    order; the runs meet in LDS (details at the kernel).
//    k_decode_tiled_mfma_sx is the same with each wave's x fetched as whole
//    token rows into a private LDS strip (runs of up to 2 groups).
#include <mutex>

#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWaves = 16;
constexpr int kBlock = 64 * kWaves;
constexpr int kWin = 2;
constexpr int kMaxCPW = 32;   // chunks per wave: K <= 32 * 16 * 32 = 16384
constexpr int kMaxTok = 4;    // tokens per pass

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                           false);
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Per-wave LDS strip for token j: kCPW chunks x 16 dwords, each 8-block stored
// as (x0,x2)(x1,x3)(x4,x6)(x5,x7); then 136*chunk sums [kM][kCPW] f32.
template <int kM, int kCPW>
struct Strip {
    static constexpr int kXBytes = kM * kCPW * 64;
    static constexpr int kBytes = kXBytes + kM * kCPW * 4;
};

template <int kM, int kCPW>
__global__ __launch_bounds__(kBlock) void k_decode_tiled(const uint16_t* __restrict__ x,
                                                         const uint8_t* __restrict__ pt,
                                                         const uint16_t* __restrict__ st,
                                                         const float* __restrict__ bias, int64_t n,
                                                         int64_t k, int tile_rows,
                                                         float* __restrict__ y) {
    using S = Strip<kM, kCPW>;
    __shared__ __attribute__((aligned(16))) uint8_t strips[kWaves][S::kBytes];
    __shared__ float part[kWaves][kM][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = blockIdx.x;
    const int64_t C = k >> 5, G = k >> 7;
    const int T = tile_rows;
    const int ln = lane < T ? lane : T - 1;  // lanes past the tile re-read its last row; never stored
    const int64_t c0 = static_cast<int64_t>(wave) * kCPW;
    uint32_t* sx = reinterpret_cast<uint32_t*>(strips[wave]);
    float* ssum = reinterpret_cast<float*>(strips[wave] + S::kXBytes);

    // this wave's x slice first (needed before any arithmetic), then the scales of
    // its groups and the first window of weight chunks.  Item = 4 values (half an
    // 8-block) of token j.
    constexpr int kItems = (kM * kCPW * 8 + kWave - 1) / kWave;
    uint2 xv[kItems];
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
        const int it = min(lane + q * kWave, kM * kCPW * 8 - 1);
        const int j = it / (kCPW * 8), r = it - j * (kCPW * 8);
        const int64_t kx = min<int64_t>(c0 * 32 + r * 4, k - 4);
        xv[q] = *reinterpret_cast<const uint2*>(x + j * k + kx);
    }
    constexpr int kGPW = (kCPW + 3) / 4;
    uint16_t sh[kGPW];
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>((c0 >> 2) + i, G - 1);
        sh[i] = st[(tile * G + g) * T + ln];
    }
    const uint8_t* wbase = pt + (tile * C * T + ln) * 16;
    u32x4 w[kWin];
#pragma unroll
    for (int i = 0; i < kWin && i < kCPW; ++i) {
        const int64_t c = min<int64_t>(c0 + i, C - 1);
        w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wbase + c * T * 16));
    }

    // stage the slice: (x0,x1),(x2,x3) -> (x0,x2),(x1,x3); the odd half of an 8-block
    // lands after the even one; 136 * chunk sums alongside
#pragma unroll
    for (int q = 0; q < kItems; ++q) {
        const int it = lane + q * kWave;
        const int itc = min(it, kM * kCPW * 8 - 1);
        const int j = itc / (kCPW * 8), r = itc - j * (kCPW * 8);
        const uint2 v = xv[q];
        // a chunk's 8 items sit in 8 aligned lanes
        const float sm = lane_group_sum<8>(bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y));
        if (it < kM * kCPW * 8) {
            *reinterpret_cast<uint2*>(sx + j * kCPW * 16 + 2 * r) =
                make_uint2((v.x & 0xFFFFu) | (v.y << 16), (v.x >> 16) | (v.y & 0xFFFF0000u));
            if ((r & 7) == 0) ssum[j * kCPW + (r >> 3)] = 136.0f * sm;
        }
    }
    // the strip is private to this wave: LDS accesses of one wave complete in order

    float acc[kM];
#pragma unroll
    for (int j = 0; j < kM; ++j) acc[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < kCPW; ++i) {
        const int slot = i % kWin;
        const uint32_t ws[4] = {w[slot].x, w[slot].y, w[slot].z, w[slot].w};
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            lo[d] = (ws[d] ^ 0x88888888u) & 0x0F0F0F0Fu;         // q+8 of k, k+2, k+4, k+6
            hi[d] = ((ws[d] >> 4) ^ 0x08888888u) & 0x0F0F0F0Fu;  // q+8 of k+1, k+3, k+5, k+7
        }
        const bool live = c0 + i < C;
        const float sc = live ? __half2float(__ushort_as_half(sh[i >> 2])) : 0.0f;
#pragma unroll
        for (int j = 0; j < kM; ++j) {
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                // strip dwords of 8-block d: (x0,x2), (x1,x3), (x4,x6), (x5,x7)
                const u32x4 xq = *reinterpret_cast<const u32x4*>(sx + j * kCPW * 16 + i * 16 + 4 * d);
                p = dot2_bf16(__builtin_amdgcn_perm(0x43434343u, lo[d], 0x04010400u), xq.x, p);
                p = dot2_bf16(__builtin_amdgcn_perm(0x43434343u, hi[d], 0x04010400u), xq.y, p);
                p = dot2_bf16(__builtin_amdgcn_perm(0x43434343u, lo[d], 0x04030402u), xq.z, p);
                p = dot2_bf16(__builtin_amdgcn_perm(0x43434343u, hi[d], 0x04030402u), xq.w, p);
            }
            acc[j] = fmaf(sc, p - ssum[j * kCPW + i], acc[j]);
        }
        if (i + kWin < kCPW) {  // compile-time: refill this slot kWin chunks ahead
            const int64_t c = min<int64_t>(c0 + i + kWin, C - 1);
            w[slot] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wbase + c * T * 16));
        }
    }

#pragma unroll
    for (int j = 0; j < kM; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    for (int i = threadIdx.x; i < kM * 64; i += kBlock) {
        const int j = i >> 6, r = i & 63;
        const int64_t row = tile * T + r;
        if (r >= T || row >= n) continue;
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) s += part[v][j][r];
        y[j * n + row] = s + (bias ? bias[row] : 0.0f);
    }
}

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// Packed dword of 8 nibbles (k .. k+7, two's complement) -> bf16 8 * (24 + q) in
// the slot order (k, k+2), (k+1, k+3), (k+4, k+6), (k+5, k+7): q + 8 in the top
// four mantissa bits of bf16 128.  The smaller offset (24 instead of the 136 of
// a low-mantissa nibble) keeps the partial sums of a group near their size.
__device__ __forceinline__ u32x4 unpack_w4_24(uint32_t w) {
    const uint32_t lo = ((w << 3) & 0x78787878u) ^ 0x40404040u;
    const uint32_t hi = ((w >> 1) & 0x78787878u) ^ 0x40404040u;
    u32x4 a;
    a.x = __builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u);
    a.y = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);
    a.z = __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u);
    a.w = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);
    return a;
}

// 8 bf16 (x0..x7) -> the slot order (x0,x2)(x1,x3)(x4,x6)(x5,x7)
__device__ __forceinline__ u32x4 pair_slots(u32x4 v) {
    u32x4 o;
    o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    return o;
}

__device__ __forceinline__ f32x4 mfma16_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// Packed dword (nibbles k..k+7, two's complement) -> bf16 136 + q in the slot
// order (k, k+4), (k+1, k+5), (k+2, k+6), (k+3, k+7): nibble pair s of the dword
// sits at bits 4s and 16 + 4s, so a shift, a mask and an xor (which turns the
// nibble into q + 8 and sets the exponent of 128) make each slot pair.
__device__ __forceinline__ u32x4 unpack_w4_136(uint32_t w) {
    u32x4 a;
    a.x = (w & 0x000F000Fu) ^ 0x43084308u;
    a.y = ((w >> 4) & 0x000F000Fu) ^ 0x43084308u;
    a.z = ((w >> 8) & 0x000F000Fu) ^ 0x43084308u;
    a.w = ((w >> 12) & 0x000F000Fu) ^ 0x43084308u;
    return a;
}

// MFMA kernel for 5..16 tokens.  Block: one tile of T = 16 kR rows; its 16 waves
// split K into runs of kGPW groups (no LDS staging of x, no barrier before the
// arithmetic: every wave issues all of its loads at once and consumes them in
// order).  Lane (r16 = l % 16, q = l / 16) holds, per group g, the 16 bytes of
// chunk 4 g + q (k in [128 g + 32 q, +32)) of row r16 of each 16-row group, and
// the same k of token r16's x (read from L2, zero past M).  MFMA step j of a
// group takes dword j of each: weights as bf16 8 * (24 + q) (unpack_w4_24),
// tokens as the other operand in the matching slot order.  One extra MFMA chain
// per group with the constant -192 as the weight operand gives -192 * sum(x)
// of the group for every token, the start value of each row group's chain, so
// the offset cancels inside the MFMA accumulator; the f16 scale is applied per
// group, the factor 1/8 at the end.  The K runs meet in LDS in a fixed order.
// Runs of 1-2 groups, and the decode FFN's down projection, take
// k_decode_tiled_mfma_sx (x staged through LDS); this one serves runs of 3-4
// groups (K up to 8192), whose x would not fit the LDS strips.
template <int kR, int kGPW>
__global__ __launch_bounds__(kBlock) void k_decode_tiled_mfma(const uint16_t* __restrict__ x, int m,
                                                              const uint8_t* __restrict__ pt,
                                                              const uint16_t* __restrict__ st,
                                                              const float* __restrict__ bias, int64_t n,
                                                              int64_t k, float* __restrict__ y) {
    constexpr int T = 16 * kR;
    __shared__ float part[kWaves][T][16];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int64_t tile = blockIdx.x;
    const int64_t C = k >> 5, G = k >> 7;
    const int64_t g0 = static_cast<int64_t>(wave) * kGPW;

    // x of token r16 (zero past m); groups past K are clamped (and skipped below)
    u32x4 xf[kGPW][4];
    const bool tok = r16 < m;
    const uint16_t* xr = x + static_cast<int64_t>(tok ? r16 : 0) * k + 32 * q;
    const int64_t gl = G - 1;
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>(g0 + i, gl);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            xf[i][j] = tok ? *reinterpret_cast<const u32x4*>(xr + g * 128 + 8 * j) : u32x4{0u, 0u, 0u, 0u};
    }
    // f16 scales of the lane's D rows 16 r + 4 q .. + 3
    uint2 sc[kGPW][kR];
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>(g0 + i, gl);
#pragma unroll
        for (int r = 0; r < kR; ++r)
            sc[i][r] = *reinterpret_cast<const uint2*>(st + (tile * G + g) * T + 16 * r + 4 * q);
    }
    // weights
    const uint8_t* wb = pt + (tile * C * T + r16) * 16;
    u32x4 w[kGPW][kR];
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>(g0 + i, gl);
#pragma unroll
        for (int r = 0; r < kR; ++r)
            w[i][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + ((4 * g + q) * T + 16 * r) * 16));
    }

    const u32x4 aoff = u32x4{0xC340C340u, 0xC340C340u, 0xC340C340u, 0xC340C340u};  // bf16 -192
    f32x4 acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        if (g0 + i >= G) break;  // wave-uniform
        u32x4 xb[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) xb[j] = pair_slots(xf[i][j]);
        f32x4 xs = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 4; ++j) xs = mfma16_bf16(aoff, xb[j], xs);
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const uint32_t ws[4] = {w[i][r].x, w[i][r].y, w[i][r].z, w[i][r].w};
            f32x4 d = xs;
#pragma unroll
            for (int j = 0; j < 4; ++j) d = mfma16_bf16(unpack_w4_24(ws[j]), xb[j], d);
            const uint32_t s01 = sc[i][r].x, s23 = sc[i][r].y;
            acc[r].x = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01))), d.x, acc[r].x);
            acc[r].y = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01 >> 16))), d.y, acc[r].y);
            acc[r].z = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23))), d.z, acc[r].z);
            acc[r].w = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23 >> 16))), d.w, acc[r].w);
        }
    }
    // lane holds D[row 16 r + 4 q + e][token r16]
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[wave][16 * r + 4 * q + e][r16] = acc[r][e];
    __syncthreads();
    for (int i = threadIdx.x; i < T * m; i += kBlock) {
        const int row = i / m, t = i - row * m;
        const int64_t grow = tile * T + row;
        if (grow >= n) continue;
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) sum += part[v][row][t];
        y[t * n + grow] = 0.125f * sum + (bias ? bias[grow] : 0.0f);
    }
}

// k_decode_tiled_mfma with x staged through LDS.  Read straight from L2 in the
// MFMA's operand layout, a wave's x fragments take 16 bytes from each of 16
// token rows per instruction (16 cache lines, half of each used), and at 16
// tokens they are as many bytes as the weights: the per-CU load path carried
// twice the weight stream.  Here each wave fetches its K slice of every token's
// x as whole rows, two groups at a time (lane l of load i of a phase: token
// i * 4 / kGP + l / (16 kGP), elements 8 (l % (16 kGP)) .. + 7 of the phase's
// slice), writes them to a private LDS strip in the slot order of the weight
// unpack (token rows padded by 16 bytes, so the 16 tokens' B reads of one MFMA
// hit distinct banks) and reads the B operands back from it.  The wave's
// partial sums go into its own strip once its loop is done.
template <int kR, int kGPW>
__global__ __launch_bounds__(kBlock) void k_decode_tiled_mfma_sx(const uint16_t* __restrict__ x, int m,
                                                                 const uint8_t* __restrict__ pt,
                                                                 const uint16_t* __restrict__ st,
                                                                 const float* __restrict__ bias, int64_t n,
                                                                 int64_t k, float* __restrict__ y) {
    static_assert(kGPW == 1 || kGPW == 2, "runs of 1 or 2 groups per wave");
    constexpr int kGP = kGPW < 2 ? kGPW : 2;  // groups per phase
    constexpr int kP = kGPW / kGP;             // phases
    constexpr int T = 16 * kR;
    constexpr int kE = 128 * kGP;       // elements of a token's phase slice
    constexpr int kRow = 2 * kE + 16;   // bytes of a token's padded strip row
    constexpr int kStrip = 16 * kRow;
    constexpr int kLPT = 16 * kGP;      // lanes per token row in a load
    constexpr int kTPI = 64 / kLPT;     // token rows per load
    constexpr int kNI = 16 / kTPI;      // loads per wave and phase
    static_assert(T * 16 * 4 <= kStrip, "a wave's partial sums fit in its strip");
    __shared__ __attribute__((aligned(16))) uint8_t strips[kWaves][kStrip];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int64_t tile = blockIdx.x;
    const int64_t C = k >> 5, G = k >> 7;
    // K split over gridDim.y blocks per tile: this block takes groups [gb, ge)
    const int64_t gh = (G + gridDim.y - 1) / gridDim.y, gb = blockIdx.y * gh, ge = min(G, gb + gh);
    const int64_t g0 = gb + static_cast<int64_t>(wave) * kGPW;
    const int64_t gl = max<int64_t>(ge - 1, 0);  // groups past the block's range are clamped (and skipped below)

    // x rows first (vmcnt retires in order), then scales, then weights
    const int e0 = 8 * (lane % kLPT);
    u32x4 xl[kP][kNI];
#pragma unroll
    for (int p = 0; p < kP; ++p)
#pragma unroll
        for (int i = 0; i < kNI; ++i) {
            const int t = i * kTPI + lane / kLPT;
            const int64_t ge0 = g0 + p * kGP;  // first group of the phase
            const bool live = t < m && ge0 + e0 / 128 < ge;
            xl[p][i] = live ? *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(t) * k + ge0 * 128 + e0)
                            : u32x4{0u, 0u, 0u, 0u};
        }
    uint2 sc[kGPW][kR];
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>(g0 + i, gl);
#pragma unroll
        for (int r = 0; r < kR; ++r)
            sc[i][r] = *reinterpret_cast<const uint2*>(st + (tile * G + g) * T + 16 * r + 4 * q);
    }
    const uint8_t* wb = pt + (tile * C * T + r16) * 16;
    u32x4 w[kGPW][kR];
#pragma unroll
    for (int i = 0; i < kGPW; ++i) {
        const int64_t g = min<int64_t>(g0 + i, gl);
#pragma unroll
        for (int r = 0; r < kR; ++r)
            w[i][r] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + ((4 * g + q) * T + 16 * r) * 16));
    }
    uint8_t* sx = strips[wave];

    // bf16 -192: minus the offset of the unpacked weights
    const u32x4 aoff = u32x4{0xC340C340u, 0xC340C340u, 0xC340C340u, 0xC340C340u};
    f32x4 acc[kR];
#pragma unroll
    for (int r = 0; r < kR; ++r) acc[r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < kP; ++p) {
        if (g0 + p * kGP >= ge) break;  // wave-uniform
#pragma unroll
        for (int i = 0; i < kNI; ++i) {
            const int t = i * kTPI + lane / kLPT;
            *reinterpret_cast<u32x4*>(sx + t * kRow + 2 * e0) = pair_slots(xl[p][i]);
        }
#pragma unroll
        for (int ii = 0; ii < kGP; ++ii) {
            const int i = p * kGP + ii;
            if (g0 + i >= ge) break;  // wave-uniform
            u32x4 xb[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xb[j] = *reinterpret_cast<const u32x4*>(sx + r16 * kRow + 2 * (128 * ii + 32 * q + 8 * j));
            f32x4 xs = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) xs = mfma16_bf16(aoff, xb[j], xs);
#pragma unroll
            for (int r = 0; r < kR; ++r) {
                const uint32_t ws[4] = {w[i][r].x, w[i][r].y, w[i][r].z, w[i][r].w};
                f32x4 d = xs;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    d = mfma16_bf16(unpack_w4_24(ws[j]), xb[j], d);
                const uint32_t s01 = sc[i][r].x, s23 = sc[i][r].y;
                acc[r].x = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01))), d.x, acc[r].x);
                acc[r].y = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01 >> 16))), d.y, acc[r].y);
                acc[r].z = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23))), d.z, acc[r].z);
                acc[r].w = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23 >> 16))), d.w, acc[r].w);
            }
        }
    }
    // lane holds D[row 16 r + 4 q + e][token r16]; part[row][token] in the wave's strip
    float* part = reinterpret_cast<float*>(sx);
#pragma unroll
    for (int r = 0; r < kR; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) part[(16 * r + 4 * q + e) * 16 + r16] = acc[r][e];
    __syncthreads();
    auto wsum = [&](int row, int t) {
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) sum += reinterpret_cast<const float*>(strips[v])[row * 16 + t];
        return sum;
    };
    for (int i = threadIdx.x; i < T * m; i += kBlock) {
        const int row = i / m, t = i - row * m;
        const int64_t grow = tile * T + row;
        if (grow >= n) continue;
        y[t * n + grow] = 0.125f * wsum(row, t) + (bias ? bias[grow] : 0.0f);
    }
}

// The decode FFN's down projection for 9-16 tokens in one launch: the 2t <= 32
// rows of h (t hi rows, then t lo rows, in slot order as the gate/up epilogue
// wrote them) are two sets of 16 columns of v_mfma_f32_16x16x32_bf16, so the
// down weights are read once per call where launches of up to 16 rows read them
// once per 8 tokens.  32-row tiles (two row groups of 16), K split over
// gridDim.y = 2 blocks per tile whose sums are added onto a y the gate/up launch
// zeroed (two addends onto zero: the same sum in either order).  Operand layout
// as in k_decode_tiled_mfma_sx: lane (r16, q) holds chunk 4 g + q of tile row
// 16 r + r16 and reads its B operands, row 16 s + r16 of set s, from an LDS
// strip of 32 rows x 256 bytes filled by global_load_lds_dwordx4: row t's
// 16-byte chunk c sits at chunk c ^ (t % 16), so the 16 rows one B read touches
// fall in distinct banks.
//
// Blocks of 8 waves (256 VGPRs per lane): each wave owns two strips and runs its
// kGPW groups with group g's rows in strip g % 2, so a group's DMAs go out two
// groups ahead (once the group that used the strip has read its B operands), and
// its weights and scales kFoldWin groups ahead.  Every load of the loop is inline
// asm (the DMAs, and the weight and scale loads into registers), so the compiler
// adds no waits there: it counts only its own loads, and a wait of its own for a
// weight would also hold the wave until the DMAs issued after that weight had
// landed.  Before group g the wave waits until g's DMAs, weights and scales have
// landed, counting the loads issued after them (fold_after); the wait names the
// group's weight and scale registers as operands, so no use of them can be
// scheduled ahead of it.
constexpr int kFoldWaves = 8;
constexpr int kFoldWin = 4;  // groups of weights and scales in flight (2 and 3: ~0.3 us slower at 8 tokens)
constexpr int kFoldLPG = 4;  // load instructions per group: 2 row groups x (scales, weights)

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Loads issued after the later of group gi's DMAs (4 instructions per set) and
// its weight and scale loads (kFoldLPG), up to the wait of group gi, in the
// kernel's issue order: DMA(0), DMA(1), LG(0 .. win-1), then for each group g
// before gi: DMA(g + 2), LG(g + win).
template <int kGPW, int kSets>
constexpr int fold_after(int gi) {
    constexpr int win = kFoldWin < kGPW ? kFoldWin : kGPW;
    int pos = 0, last = 0;
    auto dma = [&](int g) {
        if (g >= kGPW) return;
        pos += 4 * kSets;
        if (g == gi && pos > last) last = pos;
    };
    auto lg = [&](int g) {
        if (g >= kGPW) return;
        pos += kFoldLPG;
        if (g == gi && pos > last) last = pos;
    };
    dma(0);
    dma(1);
    for (int g = 0; g < win; ++g) lg(g);
    for (int g = 0; g < gi; ++g) {
        dma(g + 2);
        lg(g + win);
    }
    return pos - last;
}

__device__ __forceinline__ void asm_load16(u32x4& d, const void* p) {
    asm volatile("global_load_dwordx4 %0, %1, off nt" : "=v"(d) : "v"(p) : "memory");
}
__device__ __forceinline__ void asm_load8(u32x2& d, const void* p) {
    asm volatile("global_load_dwordx2 %0, %1, off" : "=v"(d) : "v"(p) : "memory");
}
template <int N>
__device__ __forceinline__ void fold_wait(u32x4& w0, u32x4& w1, u32x2& s0, u32x2& s1) {
    static_assert(N >= 0 && N < 64, "vmcnt counts 0..63");
    asm volatile("s_waitcnt vmcnt(%4)" : "+v"(w0), "+v"(w1), "+v"(s0), "+v"(s1) : "n"(N) : "memory");
}

template <int kGPW, int kSets>
__global__ __launch_bounds__(kFoldWaves * 64) void k_decode_fold32(const uint16_t* __restrict__ h, int rows,
                                                                   const uint8_t* __restrict__ pt,
                                                                   const uint16_t* __restrict__ st, int64_t n,
                                                                   int64_t k, float* __restrict__ y) {
    static_assert(kGPW >= 1 && kGPW <= 8, "1..8 groups per wave");
    static_assert(kSets == 1 || kSets == 2, "one or two sets of 16 rows of h");
    constexpr int kR = 2, T = 32;
    constexpr int kHR = 16 * kSets;  // rows of h (MFMA columns)
    constexpr int kStrip = kHR * 256;
    constexpr int kWin = kFoldWin < kGPW ? kFoldWin : kGPW;
    static_assert(T * kHR * 4 <= kStrip, "a wave's partial sums fit in its strip");
    static_assert(fold_after<kGPW, kSets>(0) < 64, "vmcnt counts 0..63");
    __shared__ __attribute__((aligned(1024))) int8_t strips[kFoldWaves][2][kStrip];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int64_t tile = blockIdx.x;
    const int64_t C = k >> 5, G = k >> 7;
    const int64_t gh = (G + gridDim.y - 1) / gridDim.y, gb = blockIdx.y * gh, ge = min(G, gb + gh);
    const int64_t g0 = gb + static_cast<int64_t>(wave) * kGPW;
    const int64_t gl = max<int64_t>(ge - 1, 0);

    // DMA i (0 .. 4 kSets - 1) of group gi moves rows 4 i .. 4 i + 3 into strip gi % 2: lane l
    // -> row 4 i + l / 16, landing at LDS chunk l % 16, from global chunk
    // (l % 16) ^ row % 16.  Rows past `rows` re-read the last row and groups past
    // the range the last group (their columns and sums are never used).
    auto dma_group = [&](int gi) {
        const uint16_t* hb = h + min<int64_t>(g0 + gi, gl) * 128;
        int8_t* sx = strips[wave][gi & 1];
#pragma unroll
        for (int i = 0; i < 4 * kSets; ++i) {
            const int t = 4 * i + (lane >> 4);
            lds_dma16(hb + static_cast<int64_t>(min(t, rows - 1)) * k + 8 * (r16 ^ (t & 15)), lds_addr(sx + 1024 * i));
        }
    };
    const uint8_t* wb = pt + (tile * C * T + r16) * 16;
    u32x2 sc[kWin][kR];
    u32x4 w[kWin][kR];
    auto load_group = [&](int gi) {  // into slot gi % kWin
        const int64_t g = min<int64_t>(g0 + gi, gl);
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            asm_load8(sc[gi % kWin][r], st + (tile * G + g) * T + 16 * r + 4 * q);
            asm_load16(w[gi % kWin][r], wb + ((4 * g + q) * T + 16 * r) * 16);
        }
    };
    dma_group(0);
    if (kGPW > 1) dma_group(1);
#pragma unroll
    for (int gi = 0; gi < kWin; ++gi) load_group(gi);
    const u32x4 aoff = u32x4{0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};  // bf16 -136
    f32x4 acc[kSets][kR];
#pragma unroll
    for (int s2 = 0; s2 < kSets; ++s2)
#pragma unroll
        for (int r = 0; r < kR; ++r) acc[s2][r] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gi = 0; gi < kGPW; ++gi) {
        if (g0 + gi >= ge) break;  // wave-uniform
        const int sl = gi % kWin;
        switch (gi) {
#define TQ_FOLD_WAIT(G)                                                                        \
    case G:                                                                                    \
        if constexpr (G < kGPW) fold_wait<fold_after<kGPW, kSets>(G)>(w[sl][0], w[sl][1], sc[sl][0], sc[sl][1]); \
        break;
            TQ_FOLD_WAIT(0)
            TQ_FOLD_WAIT(1)
            TQ_FOLD_WAIT(2)
            TQ_FOLD_WAIT(3)
            TQ_FOLD_WAIT(4)
            TQ_FOLD_WAIT(5)
            TQ_FOLD_WAIT(6)
            TQ_FOLD_WAIT(7)
#undef TQ_FOLD_WAIT
        }
        const int8_t* sx = strips[wave][gi & 1];
        u32x4 xb[kSets][4];
#pragma unroll
        for (int s2 = 0; s2 < kSets; ++s2)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                xb[s2][j] = *reinterpret_cast<const u32x4*>(sx + (16 * s2 + r16) * 256 + (((4 * q + j) ^ r16) << 4));
        if (gi + 2 < kGPW) {
            // every read of this strip has returned: group gi + 2 may land in it
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            dma_group(gi + 2);
        }
        f32x4 xs[kSets];
#pragma unroll
        for (int s2 = 0; s2 < kSets; ++s2) {
            xs[s2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 4; ++j) xs[s2] = mfma16_bf16(aoff, xb[s2][j], xs[s2]);
        }
#pragma unroll
        for (int r = 0; r < kR; ++r) {
            const u32x4 wv = w[sl][r];
            const uint32_t ws[4] = {wv.x, wv.y, wv.z, wv.w};
            f32x4 d[kSets];
#pragma unroll
            for (int s2 = 0; s2 < kSets; ++s2) d[s2] = xs[s2];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 a = unpack_w4_136(ws[j]);
#pragma unroll
                for (int s2 = 0; s2 < kSets; ++s2) d[s2] = mfma16_bf16(a, xb[s2][j], d[s2]);
            }
            const uint32_t s01 = sc[sl][r].x, s23 = sc[sl][r].y;
            const float sv[4] = {__half2float(__ushort_as_half(static_cast<uint16_t>(s01))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s01 >> 16))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s23))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s23 >> 16)))};
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int s2 = 0; s2 < kSets; ++s2) acc[s2][r][e] = fmaf(sv[e], d[s2][e], acc[s2][r][e]);
        }
        // this group's weights and scales are consumed: their slot takes group gi + kWin
        if (gi + kWin < kGPW) load_group(gi + kWin);
    }
    // no DMA into the strips is still in flight (a wave past its range issued some),
    // and every read of them has returned: the partial sums go to strip 0,
    // part[row][column], lane holding D[row 16 r + 4 q + e][column 16 s + r16].
    // A wave that left the loop early still has weight and scale loads in flight
    // into registers that are dead on that path: the compiler would be free to
    // place other values there before the wait, and the landing loads would
    // overwrite them.  Every slot is an operand of the final wait, so all of them
    // stay allocated until it.
#pragma unroll
    for (int s2 = 0; s2 < kWin; ++s2) fold_wait<0>(w[s2][0], w[s2][1], sc[s2][0], sc[s2][1]);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    float* part = reinterpret_cast<float*>(strips[wave][0]);
#pragma unroll
    for (int s2 = 0; s2 < kSets; ++s2)
#pragma unroll
        for (int r = 0; r < kR; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) part[(16 * r + 4 * q + e) * kHR + 16 * s2 + r16] = acc[s2][r][e];
    __syncthreads();
    auto wsum = [&](int row, int c) {
        float sum = 0.0f;
#pragma unroll
        for (int v = 0; v < kFoldWaves; ++v) sum += reinterpret_cast<const float*>(strips[v][0])[row * kHR + c];
        return sum;
    };
    const int tt = rows >> 1;
    for (int i = threadIdx.x; i < T * tt; i += kFoldWaves * 64) {
        const int row = i / tt, t = i - row * tt;
        const int64_t grow = tile * T + row;
        if (grow >= n) continue;
        const float v = wsum(row, t) + wsum(row, tt + t);
        if (gridDim.y == 1)
            y[t * n + grow] = v;
        else
            atomicAdd(&y[t * n + grow], v);
    }
}

// Decode kernel for 1..kM tokens (kM * kR <= 16), T = 16 kR rows per tile.
//
// Lane l (i = l % 16, kg = l / 16) loads, per step, the 16 bytes of row
// 16 (kg % kR) + i at chunk kS step + kg / kR (kS = 4 / kR chunks per step, kR
// steps per 128-element group), and feeds each of their 4 dwords to one MFMA as
// row i of k-group kg.  B lane (kg, c) holds the matching 8 values of token
// c / kR when c % kR == kg % kR and c / kR < kM, zeros otherwise.  Then
//   D[i][c] = sum over the kS chunks of the step of
//             row 16 (c % kR) + i  .  x_{c / kR}
// and a lane of the output holds D[4 (l / 16) + e][l % 16], e = 0..3: four
// consecutive tile rows of one token.  The accumulators restart per group; the
// group's f16 scale and 136 * sum(x) of the group are applied as
// y += s * (acc - 136 X_g).
//
// Each wave stages its K slice of every token's x in a private LDS strip (slot
// order as above; a zero strip of the same size serves the other B lanes) and
// keeps 136 X_g per (token, group) in registers.  The caller's x is put in slot
// order and summed on the way (DPP, no LDS round trips); the down projection's x
// (kEpiFold) is h as kEpiGateUp wrote it, already in slot order with the sums
// of its 32-column blocks beside it, and is copied as it is.  Loads are issued x first,
// then scales, then kWin steps of weights ahead of the arithmetic (in-order
// vmcnt), and every wave runs all its groups (groups past K read clamped
// addresses with a zero scale) so the refills are not moved behind a branch.
// The 16 waves' partial sums meet in LDS in a fixed order.
// What the block does with its rows' dot products (16 waves summed in order):
//  kEpiPlain:  y[j][row] = sum + bias[row] for the m tokens.
//  kEpiFold:   the m = 2t tokens are t rows and their t low parts (an f32 input
//              split into bf16 hi + lo); y[j][row] = sum_j + sum_{t+j} + bias[row].
//  kEpiGateUp: the 64-row tile holds gate rows 32 tile .. + 31 (rows 0-31) and
//              the up rows of the same indices (rows 32-63) of a Llama FFN;
//              h = g / (1 + exp(-g)) * u goes out as bf16 hi = bf16(h) and lo =
//              bf16(h - hi) into the down projection's input rows (see MlpRows),
//              in slot order (h_slot), and the f32 sums of the tile's 32 hi and
//              32 lo values to xsum[row][tile].
enum DiagEpi { kEpiPlain = 0, kEpiFold = 1, kEpiGateUp = 2 };

// Position of h column c in its row: 8-blocks in slot order, columns 8b + e at
// 8b + 2e (e < 4) and 8b + 2(e - 4) + 1 (e >= 4).
__host__ __device__ inline int64_t h_slot(int64_t c) { return (c & ~int64_t{7}) | ((c & 3) << 1) | ((c >> 2) & 1); }

// Decode FFN workspace: the 2m bf16 rows of h (hi and lo of each token), then
// the f32 sums of their 32-column blocks, [2m][F / 32].
constexpr int64_t round_up256(int64_t b) { return (b + 255) / 256 * 256; }
constexpr int64_t mlp_h_bytes(int64_t m, int64_t f) { return round_up256(2 * m * f * 2); }

// Rows of the down projection's bf16 input for token J of an m-token FFN, in
// groups of q tokens (q = 2, 4 or 8; one down launch per group): group c = J / q
// with t = min(q, m - q c) tokens occupies rows 2 q c .. 2 q c + 2t - 1 as (hi of
// its tokens, lo of its tokens), so each group is one launch of 2t contiguous
// rows; for m <= q that is the m hi rows, then the m lo rows.
struct MlpRows {
    __host__ __device__ static int64_t hi(int64_t j, int64_t m, int q) { return 2 * q * (j / q) + (j % q); }
    __host__ __device__ static int64_t lo(int64_t j, int64_t m, int q) {
        const int64_t c = j / q, t = m - q * c < q ? m - q * c : q;
        return 2 * q * c + t + (j % q);
    }
};

// Epilogues shared by the diagonal kernels; wsum(j, r) is the block's dot
// product of token j with tile row r (the waves' partial sums added in order).
template <class WSum>
__device__ __forceinline__ void plain_epilogue(const WSum& wsum, int m, int T, int64_t tile, int64_t n,
                                               const float* bias, float* y) {
    for (int i = threadIdx.x; i < m * T; i += kBlock) {
        const int j = i / T, r = i - j * T;
        const int64_t row = tile * T + r;
        if (row >= n) continue;
        y[j * n + row] = wsum(j, r) + (bias ? bias[row] : 0.0f);
    }
}

// kEpiGateUp for m <= 16 tokens of a 64-row gate/up tile (n = 2f stacked rows),
// run by the threads whose index in the tile's thread range is i (a range starts
// at a multiple of 64 threads).
template <class WSum>
__device__ __forceinline__ void gate_up_h(const WSum& wsum, int m, int64_t tile, int64_t n, uint16_t* hout,
                                          float* xsum, int tok0, int mtot, int rows_group, int i) {
    const int64_t f = n >> 1;  // h columns: the stacked weight has 2f rows, f % 32 == 0
    const int lane = threadIdx.x & 63;
    // thread i < 32 m: token i / 32, column 32 tile + i % 32, so that the 32
    // columns of a token are one half of a wave (two whole DPP rows)
    if (i < m * 32) {
        const int j = i >> 5, r = i & 31;
        const int64_t hc = tile * 32 + r;
        const float g = wsum(j, r), u = wsum(j, 32 + r);
        const float h = g * (1.0f / (1.0f + __expf(-g))) * u;
        const __bf16 hi = static_cast<__bf16>(h);
        const __bf16 lo = static_cast<__bf16>(h - static_cast<float>(hi));
        const int64_t J = tok0 + j, rh = MlpRows::hi(J, mtot, rows_group), rl = MlpRows::lo(J, mtot, rows_group);
        hout[rh * f + h_slot(hc)] = __builtin_bit_cast(uint16_t, hi);
        hout[rl * f + h_slot(hc)] = __builtin_bit_cast(uint16_t, lo);
        const int sh = __float_as_int(lane_group_sum<16>(static_cast<float>(hi)));
        const int sl = __float_as_int(lane_group_sum<16>(static_cast<float>(lo)));
        auto half_sum = [&](int v) {  // rows 0 + 1 for lanes 0-31, rows 2 + 3 for lanes 32-63
            const float a = __int_as_float(__builtin_amdgcn_readlane(v, 0)) +
                            __int_as_float(__builtin_amdgcn_readlane(v, 16));
            const float b = __int_as_float(__builtin_amdgcn_readlane(v, 32)) +
                            __int_as_float(__builtin_amdgcn_readlane(v, 48));
            return lane < 32 ? a : b;
        };
        const float th = half_sum(sh), tl = half_sum(sl);
        if (r == 0) {
            xsum[rh * (f >> 5) + tile] = th;
            xsum[rl * (f >> 5) + tile] = tl;
        }
    }
}

// The output a K-split down projection accumulates into, zeroed by the grid.
__device__ __forceinline__ void zero_grid(float* yz, int64_t yz_n) {
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; q < yz_n;
         q += static_cast<int64_t>(gridDim.x) * kBlock)
        yz[q] = 0.0f;
}

template <class WSum>
__device__ __forceinline__ void gate_up_epilogue(const WSum& wsum, int m, int64_t tile, int64_t n, uint16_t* hout,
                                                 float* xsum, int tok0, int mtot, int rows_group, float* yz,
                                                 int64_t yz_n) {
    gate_up_h(wsum, m, tile, n, hout, xsum, tok0, mtot, rows_group, static_cast<int>(threadIdx.x));
    zero_grid(yz, yz_n);
}

template <int kR, int kM, int kGPW, int kWinD, int kEpi>
__global__ __launch_bounds__(kBlock) void k_decode_diag(const uint16_t* __restrict__ x, int m,
                                                        const uint8_t* __restrict__ pt,
                                                        const uint16_t* __restrict__ st,
                                                        const float* __restrict__ bias, int64_t n, int64_t k,
                                                        float* __restrict__ y, uint16_t* __restrict__ hout,
                                                        float* __restrict__ xsum, int tok0, int mtot, int rows_group,
                                                        float* __restrict__ yz, int64_t yz_n) {
    static_assert(kM * kR <= 16, "columns are (token, row group) pairs");
    static_assert(kEpi != kEpiGateUp || kR == 4, "gate/up tiles are 64 rows");
    constexpr int T = 16 * kR;
    constexpr int kS = 4 / kR;                  // chunks per step
    constexpr int kCPW = 4 * kGPW;              // chunks per wave
    constexpr int kSteps = kCPW / kS;           // weight loads per lane
    constexpr int kStrip = kCPW * 64;           // bytes of one token's slice (bf16)
    constexpr bool kPre = kEpi == kEpiFold;     // x in slot order with its block sums
    constexpr int kItems = kM * kCPW * (kPre ? 4 : 8);  // 8- (kPre) or 4-element items
    constexpr int kIPL = (kItems + kWave - 1) / kWave;
    constexpr int kW = kWinD < kSteps ? kWinD : kSteps;
    // token strips padded by 16 bytes: unpadded, the tokens' B-operand reads of one
    // MFMA (strips 2^n bytes apart) fell in the same LDS banks, an 8-way conflict at
    // 8 x rows
    __shared__ __attribute__((aligned(16))) uint8_t xs[kWaves][kM][kStrip + 16];
    __shared__ __attribute__((aligned(16))) uint8_t zs[kStrip];  // zeros, written by every wave
    __shared__ __attribute__((aligned(16))) float part[kWaves][kM][T];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = blockIdx.x;
    const int64_t C = k >> 5, G = k >> 7;
    // K split over gridDim.y blocks per tile: this block takes groups [gb, ge)
    const int64_t gh = (G + gridDim.y - 1) / gridDim.y, gb = blockIdx.y * gh, ge = min(G, gb + gh);
    const int64_t g0 = gb + static_cast<int64_t>(wave) * kGPW, c0 = 4 * g0;
    const int col = lane & 15, kg = lane >> 4;
    const int rg = kg % kR, cs = kg / kR;  // this lane's row group and chunk slot (loads)
    const int tok = col / kR;              // token of this lane's output column
    const int row0 = 16 * (col % kR) + 4 * kg;  // first of its four output rows

    // x items: item it -> token it / (8 kCPW), elements 4 (it % (8 kCPW)) .. + 3 of
    // the wave's slice (clamped past K; zero past m).  kPre: token it / (4 kCPW),
    // elements 8 (it % (4 kCPW)) .. + 7, and tokens past m repeat token m - 1 (their
    // output columns are never stored); xsb: the 32-column sums of the wave's
    // groups, item it -> token it / (4 kGPW), block it % (4 kGPW) of the slice.
    using XItem = std::conditional_t<kPre, u32x4, uint2>;
    XItem xv[kIPL];
    constexpr int kSItems = kM * kGPW * 4, kSPL = (kSItems + kWave - 1) / kWave;
    float xsb[kPre ? kSPL : 1];
#pragma unroll
    for (int q = 0; q < kIPL; ++q) {
        const int it = min(lane + kWave * q, kItems - 1);
        if constexpr (kPre) {
            const int j = it / (kCPW * 4), r = it - j * (kCPW * 4);
            const int64_t kx = min<int64_t>(c0 * 32 + 8 * r, ge * 128 - 8);
            xv[q] = *reinterpret_cast<const u32x4*>(x + min(j, m - 1) * k + kx);
        } else {
            const int j = it / (kCPW * 8), r = it - j * (kCPW * 8);
            const int64_t kx = min<int64_t>(c0 * 32 + 4 * r, ge * 128 - 4);
            xv[q] = j < m ? *reinterpret_cast<const uint2*>(x + j * k + kx) : make_uint2(0u, 0u);
        }
    }
    if constexpr (kPre) {
#pragma unroll
        for (int q = 0; q < kSPL; ++q) {
            const int it = min(lane + kWave * q, kSItems - 1);
            const int j = it / (4 * kGPW), b = it - j * (4 * kGPW);
            xsb[q] = xsum[min(j, m - 1) * (k >> 5) + 4 * min<int64_t>(g0 + (b >> 2), ge - 1) + (b & 3)];
        }
    }
    uint2 sc[kGPW];
#pragma unroll
    for (int g = 0; g < kGPW; ++g)
        sc[g] = *reinterpret_cast<const uint2*>(st + (tile * G + min<int64_t>(g0 + g, ge - 1)) * T + row0);
    const uint8_t* wb = pt + (tile * C * T + 16 * rg + (lane & 15)) * 16;
    u32x4 w[kW];
#pragma unroll
    for (int i = 0; i < kW; ++i)
        w[i] = __builtin_nontemporal_load(
            reinterpret_cast<const u32x4*>(wb + min<int64_t>(c0 + i * kS + cs, 4 * ge - 1) * T * 16));

    // every wave zeroes the shared zero strip (the same value from every writer, so
    // no barrier is needed before a wave reads what it wrote itself)
    for (int b = lane * 16; b < kStrip; b += kWave * 16) *reinterpret_cast<u32x4*>(&zs[b]) = u32x4{0u, 0u, 0u, 0u};
    float corr[kGPW];
    if constexpr (kPre) {
#pragma unroll
        for (int q = 0; q < kIPL; ++q) {
            const int it = lane + kWave * q;
            const int j = it / (kCPW * 4), r = it - j * (kCPW * 4);
            if (it < kItems) *reinterpret_cast<u32x4*>(&xs[wave][j][r * 16]) = xv[q];
        }
        // a group's four block sums sit in 4 aligned lanes
        float gsum[kSPL];
#pragma unroll
        for (int q = 0; q < kSPL; ++q) gsum[q] = lane_group_sum<4>(xsb[q]);
#pragma unroll
        for (int g = 0; g < kGPW; ++g) {
            float c = 0.0f;
#pragma unroll
            for (int j = 0; j < kM; ++j) {
                const int it = j * 4 * kGPW + 4 * g;  // first block of (token j, group g)
                const float v = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gsum[it / kWave]), it % kWave));
                c = tok == j ? v : c;
            }
            corr[g] = 136.0f * c;
        }
    } else {
        // stage: lanes 2b, 2b+1 hold an 8-block's (x0..x3) and (x4..x7); the even lane
        // writes slots (x0,x4)(x1,x5), the odd lane (x2,x6)(x3,x7)
        float gsum[kIPL];
#pragma unroll
        for (int q = 0; q < kIPL; ++q) {
            const int it = lane + kWave * q;
            const int itc = min(it, kItems - 1);
            const int j = itc / (kCPW * 8), r = itc - j * (kCPW * 8);
            const uint2 v = xv[q];
            const uint2 p = make_uint2(dpp_u32<kDppXor1>(v.x), dpp_u32<kDppXor1>(v.y));
            const bool odd = r & 1;
            const uint32_t hi = odd ? v.y : p.x, lo = odd ? p.y : v.x;
            if (it < kItems)
                *reinterpret_cast<uint2*>(&xs[wave][j][(r >> 1) * 16 + (odd ? 8 : 0)]) = make_uint2(
                    __builtin_amdgcn_perm(hi, lo, 0x05040100u), __builtin_amdgcn_perm(hi, lo, 0x07060302u));
            // a group is 32 consecutive items (half the wave): the sums of its two
            // 16-lane rows
            gsum[q] = lane_group_sum<16>(bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y));
        }
#pragma unroll
        for (int g = 0; g < kGPW; ++g) {
            float c = 0.0f;
#pragma unroll
            for (int j = 0; j < kM; ++j) {
                const int it = j * kCPW * 8 + 32 * g;  // first item of (token j, group g)
                const int src = __float_as_int(gsum[it / kWave]);
                const float v = __int_as_float(__builtin_amdgcn_readlane(src, it % kWave)) +
                                __int_as_float(__builtin_amdgcn_readlane(src, it % kWave + 16));
                c = tok == j ? v : c;
            }
            corr[g] = 136.0f * c;
        }
    }
    const bool diag = col % kR == rg && tok < kM;
    const uint8_t* bsrc = diag ? &xs[wave][tok][cs * 64] : &zs[0];
    // the strips are private to the wave: its LDS accesses complete in order

    f32x4 tot = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < kGPW; ++g) {
        const bool live = g0 + g < ge;
        f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll
        for (int ss = 0; ss < kR; ++ss) {
            const int i = kR * g + ss;  // step
            const int slot = i % kW;
            const uint32_t ws[4] = {w[slot].x, w[slot].y, w[slot].z, w[slot].w};
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const u32x4 b = *reinterpret_cast<const u32x4*>(bsrc + (i * kS * 4 + d) * 16);
                if (d & 1)
                    a1 = mfma16_bf16(unpack_w4_136(ws[d]), b, a1);
                else
                    a0 = mfma16_bf16(unpack_w4_136(ws[d]), b, a0);
            }
            if (i + kW < kSteps) {
                w[slot] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(wb + min<int64_t>(c0 + (i + kW) * kS + cs, 4 * ge - 1) * T * 16));
                __builtin_amdgcn_sched_barrier(0);  // the refill is issued here, not after the group
            }
        }
        const uint32_t s01 = live ? sc[g].x : 0u, s23 = live ? sc[g].y : 0u;
        tot.x = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01))), (a0.x + a1.x) - corr[g], tot.x);
        tot.y = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s01 >> 16))), (a0.y + a1.y) - corr[g], tot.y);
        tot.z = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23))), (a0.z + a1.z) - corr[g], tot.z);
        tot.w = fmaf(__half2float(__ushort_as_half(static_cast<uint16_t>(s23 >> 16))), (a0.w + a1.w) - corr[g], tot.w);
    }
    if (tok < kM) *reinterpret_cast<f32x4*>(&part[wave][tok][row0]) = tot;
    __syncthreads();
    auto wsum = [&](int j, int r) {
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) s += part[v][j][r];
        return s;
    };
    if constexpr (kEpi == kEpiPlain) {
        plain_epilogue(wsum, m, T, tile, n, bias, y);
    } else if constexpr (kEpi == kEpiFold) {
        const int t = m >> 1;
        for (int i = threadIdx.x; i < t * T; i += kBlock) {
            const int j = i / T, r = i - j * T;
            const int64_t row = tile * T + r;
            if (row >= n) continue;
            const float v = (wsum(j, r) + wsum(t + j, r)) + (bias && blockIdx.y == 0 ? bias[row] : 0.0f);
            if (gridDim.y == 1)
                y[j * n + row] = v;
            else  // K halves onto a zeroed y: two addends onto zero, the same sum in either order
                atomicAdd(&y[j * n + row], v);
        }
    } else {
        gate_up_epilogue(wsum, m, tile, n, hout, xsum, tok0, mtot, rows_group, yz, yz_n);
    }
}

// The FFN's gate/up at 5-16 tokens on v_mfma_f32_16x16x32_bf16: the MFMA's 16
// columns are the 16 token slots (tokens past m are zero rows of x), so every
// MFMA column carries a token.  A block of 16 waves takes kTPB consecutive
// 64-row tiles (gate rows 0-31, up rows 32-63 of each) with one staging of x;
// its waves split K into runs of kGPW groups.  Lane (r16, q) holds, per
// (tile, group) step and row block rb, the 16 bytes of chunk 4 g + q of tile row
// 16 rb + r16; dword d is the A operand of MFMA d of that row block (row r16,
// k-group q).  Its B operand for MFMA d is token r16's 8-block 4 (4 g + q) + d of
// the wave's x slice in slot order (the unpack's order), read from the wave's LDS
// strip and shared by the 4 row blocks; the output lane holds D[tile row 16 rb +
// 4 q + e][token r16].  The accumulators restart per step from -136 X_g (X_g the
// token's sum over the group: four MFMAs of the step's B operands against bf16
// -136, shared by the row blocks), and the step's f16 row scales are applied as
// tot += s * acc.
//
// x staging: each lane loads 16-byte 8-blocks of its tokens' slices (tokens past
// m read as zeros), puts each in slot order with four byte permutes and writes it
// to the token's strip (padded by 16 bytes, so the 16 rows of one B read fall in
// distinct banks).  Weights and scales run kGuWin steps ahead
// of the arithmetic.  The waves' partial sums meet in LDS in a fixed order (over
// the wave's dead strips), and the epilogue of tile tt runs on threads [512 tt,
// 512 tt + 32 m).  With 448 tiles (F = 14336) two tiles per block make 224
// blocks, one round on 256 CUs.
constexpr int kGuWin = 2;  // (tile, group) steps of weights and scales in flight

template <int kGPW, int kTPB>
__global__ __launch_bounds__(kBlock) void k_decode_gu16(const uint16_t* __restrict__ x, int m,
                                                        const uint8_t* __restrict__ pt,
                                                        const uint16_t* __restrict__ st, int64_t n, int64_t k,
                                                        uint16_t* __restrict__ hout, float* __restrict__ xsum,
                                                        int tok0, int mtot, int rows_group, float* __restrict__ yz,
                                                        int64_t yz_n) {
    static_assert(kTPB == 1 || kTPB == 2, "one or two tiles per block");
    constexpr int kM = 16, T = 64, kRB = T / 16;
    constexpr int kCPW = 4 * kGPW;      // chunks per wave
    constexpr int kStrip = kCPW * 64;   // bytes of one token's slice (bf16)
    constexpr int kStripP = kStrip + 16;
    constexpr int kBPT = 4 * kCPW;      // 8-blocks of a token's slice
    constexpr int kItems = kM * kBPT;
    static_assert(kItems % kWave == 0 && kBPT % 16 == 0, "whole loads; a group is one 16-lane row");
    constexpr int kIPL = kItems / kWave;
    constexpr int kSteps = kTPB * kGPW;  // (tile, group) steps of the block
    constexpr int kWin = kGuWin < kSteps ? kGuWin : kSteps;
    // a wave's region: its token strips (strip j at j kStripP), later its partial sums
    constexpr int kRegion = kM * kStripP > kTPB * kM * T * 4 ? kM * kStripP : kTPB * kM * T * 4;
    static_assert(kTPB * 512 <= kBlock && kM * 32 <= 512, "a tile's epilogue takes 32 m of its 512 threads");
    __shared__ __attribute__((aligned(16))) uint8_t xs[kWaves][kRegion];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int r16 = lane & 15, q = lane >> 4;
    const int64_t tiles = (n + T - 1) / T;
    const int64_t tile0 = static_cast<int64_t>(blockIdx.x) * kTPB;
    const int64_t C = k >> 5, G = k >> 7;
    const int64_t g0 = static_cast<int64_t>(wave) * kGPW, c0 = 4 * g0;

    // x items: item it -> token it / kBPT, elements 8 (it % kBPT) .. + 7 of the
    // wave's slice (clamped past K; zero past m)
    u32x4 xv[kIPL];
#pragma unroll
    for (int i = 0; i < kIPL; ++i) {
        const int it = lane + kWave * i;
        const int j = it / kBPT, b = it - j * kBPT;
        const int64_t kx = min<int64_t>(c0 * 32 + 8 * b, k - 8);
        xv[i] = j < m ? *reinterpret_cast<const u32x4*>(x + j * k + kx) : u32x4{0u, 0u, 0u, 0u};
    }
    // step s: tile tile0 + s / kGPW (clamped to the last tile), group g0 + s % kGPW
    // (clamped to the last group; past K the scale is zero below)
    uint2 sc[kWin][kRB];
    u32x4 w[kWin][kRB];
    auto load_step = [&](int s) {  // into slot s % kWin
        const int64_t t = min<int64_t>(tile0 + s / kGPW, tiles - 1), g = min<int64_t>(g0 + s % kGPW, G - 1);
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) {
            sc[s % kWin][rb] = *reinterpret_cast<const uint2*>(st + (t * G + g) * T + 16 * rb + 4 * q);
            w[s % kWin][rb] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(pt + ((t * C + 4 * g + q) * T + 16 * rb + r16) * 16));
        }
    };
#pragma unroll
    for (int s = 0; s < kWin; ++s) load_step(s);

    // stage: a lane's 8-block (x0..x7) goes to its strip as (x0,x4)(x1,x5)(x2,x6)(x3,x7)
#pragma unroll
    for (int i = 0; i < kIPL; ++i) {
        const int it = lane + kWave * i;
        const int j = it / kBPT, b = it - j * kBPT;
        const u32x4 v = xv[i];
        *reinterpret_cast<u32x4*>(&xs[wave][j * kStripP + b * 16]) =
            u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                  __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
    }
    // the strips are private to the wave: its LDS accesses complete in order
    const uint8_t* bsrc = &xs[wave][r16 * kStripP];
    // bf16 -136 in every A entry: the MFMAs over a group's B operands give -136 x
    // (the token's sum over the group) in every row, the start of each row block's sums
    const u32x4 aoff = u32x4{0xC308C308u, 0xC308C308u, 0xC308C308u, 0xC308C308u};

    f32x4 tot[kTPB][kRB];
#pragma unroll
    for (int tt = 0; tt < kTPB; ++tt)
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) tot[tt][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kSteps; ++s) {
        const int tt = s / kGPW, g = s % kGPW;
        const bool live = g0 + g < G;
        u32x4 bx[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) bx[d] = *reinterpret_cast<const u32x4*>(bsrc + (16 * g + 4 * q + d) * 16);
        f32x4 xoff = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < 4; ++d) xoff = mfma16_bf16(aoff, bx[d], xoff);
        f32x4 acc[kRB];
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) acc[rb] = xoff;
        const int slot = s % kWin;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int rb = 0; rb < kRB; ++rb) {
                const u32x4 wv = w[slot][rb];
                const uint32_t wd = d == 0 ? wv.x : (d == 1 ? wv.y : (d == 2 ? wv.z : wv.w));
                acc[rb] = mfma16_bf16(unpack_w4_136(wd), bx[d], acc[rb]);
            }
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb) {
            const uint32_t s01 = live ? sc[slot][rb].x : 0u, s23 = live ? sc[slot][rb].y : 0u;
            const float sv[4] = {__half2float(__ushort_as_half(static_cast<uint16_t>(s01))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s01 >> 16))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s23))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(s23 >> 16)))};
#pragma unroll
            for (int e = 0; e < 4; ++e) tot[tt][rb][e] = fmaf(sv[e], acc[rb][e], tot[tt][rb][e]);
        }
        if (s + kWin < kSteps) {
            load_step(s + kWin);
            __builtin_amdgcn_sched_barrier(0);  // the refill is issued here, not at its use
        }
    }
    // this wave's strips are dead: its partial sums, [tile][token][tile row] f32, go there
    float* part = reinterpret_cast<float*>(&xs[wave][0]);
#pragma unroll
    for (int tt = 0; tt < kTPB; ++tt)
#pragma unroll
        for (int rb = 0; rb < kRB; ++rb)
            *reinterpret_cast<f32x4*>(&part[(tt * kM + r16) * T + 16 * rb + 4 * q]) = tot[tt][rb];
    __syncthreads();
    const int tt = kTPB == 1 ? 0 : static_cast<int>(threadIdx.x >> 9);  // wave-uniform
    auto wsum = [&](int j, int r) {
        float s = 0.0f;
#pragma unroll
        for (int v = 0; v < kWaves; ++v) s += reinterpret_cast<const float*>(&xs[v][0])[(tt * kM + j) * T + r];
        return s;
    };
    if (tile0 + tt < tiles)
        gate_up_h(wsum, m, tile0 + tt, n, hout, xsum, tok0, mtot, rows_group,
                  static_cast<int>(threadIdx.x) - 512 * tt);
    zero_grid(yz, yz_n);
}

// kR in {1, 2, 4}; kM in {1, 2, 4} (3 tokens run as 4 with a zero token); groups per
// wave 1..8 (K <= 16384)
struct DiagArgs {
    const uint16_t* x;
    int m;
    const uint8_t* pt;
    const uint16_t* st;
    const float* b;
    int64_t n, k;
    float* y;
    uint16_t* hout;  // kEpiGateUp
    int tok0, mtot;  // kEpiGateUp
    int rows_group = 2;      // kEpiGateUp: tokens per MlpRows group
    float* xsum = nullptr;   // kEpiGateUp: h's 32-column sums out; kEpiFold: x's in
    float* yz = nullptr;     // kEpiGateUp: zeroed (yz_n floats)
    int64_t yz_n = 0;
    int ksplit = 1;          // kEpiFold only: blocks per tile along K; their sums are
                             // added into y atomically, so the caller zeroes y first
                             // (the gate/up launch of the same FFN does, through yz)
};

template <int kR, int kM, int kEpi>
int launch_diag(int64_t gpw, int64_t tiles, hipStream_t s, const DiagArgs& a) {
    constexpr int kWinD = kR == 1 ? 2 : 3;  // measured: steps of 4 chunks want a shorter window
    // only the fold epilogue adds K parts; the others would store one part over another
    if (a.ksplit < 1 || (a.ksplit > 1 && kEpi != kEpiFold))
        return fail(TQ_EINVAL, "tq_gemv_w4g128_tiled: K split %d needs the accumulating epilogue", a.ksplit);
    if (kEpi == kEpiFold && (!a.xsum || !aligned(a.xsum, 16) || !aligned(a.x, 16) || a.k % 128 != 0))
        return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: h rows and their sums must be 16-byte aligned");
    if (kEpi == kEpiGateUp && (!a.xsum || !aligned(a.xsum, 4)))
        return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: no place for the block sums of h");
    const dim3 grid(static_cast<unsigned>(tiles), static_cast<unsigned>(a.ksplit));
#define TQ_DIAG(G)                                                                                      \
    k_decode_diag<kR, kM, G, kWinD, kEpi><<<grid, kBlock, 0, s>>>(a.x, a.m, a.pt, a.st, a.b, a.n, a.k, a.y, \
                                                                  a.hout, a.xsum, a.tok0, a.mtot,           \
                                                                  a.rows_group, a.yz, a.yz_n)
    // the exact groups per wave, so that no wave of the block runs dead groups (K =
    // 14336, the Llama FFN's intermediate size, is 7 per wave)
    switch (gpw) {
        case 1: TQ_DIAG(1); break;
        case 2: TQ_DIAG(2); break;
        case 3: TQ_DIAG(3); break;
        case 4: TQ_DIAG(4); break;
        default:
            // 8 x rows fit the LDS at up to 4 groups per wave only
            if constexpr (kM <= 4) {
                switch (gpw) {
                    case 5: TQ_DIAG(5); break;
                    case 6: TQ_DIAG(6); break;
                    case 7: TQ_DIAG(7); break;
                    default: TQ_DIAG(8); break;
                }
            } else {
                return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: %lld groups per wave for 8 rows", (long long)gpw);
            }
    }
#undef TQ_DIAG
    return check_launch("tq_gemv_w4g128_tiled");
}

template <int kR, int kEpi>
int launch_diag_m(int64_t gpw, int64_t tiles, hipStream_t s, const DiagArgs& a) {
    if (a.m == 1) return launch_diag<kR, 1, kEpi>(gpw, tiles, s, a);
    if (a.m == 2) return launch_diag<kR, 2, kEpi>(gpw, tiles, s, a);
    if constexpr (kR <= 2 && kEpi == kEpiFold)
        if (a.m > 4) return launch_diag<kR, 8, kEpi>(gpw, tiles, s, a);  // 3-4 tokens' hi and lo rows
    return launch_diag<kR, 4, kEpi>(gpw, tiles, s, a);
}

// The 16x16x32 gate/up kernel for 5-16 tokens, at most 2 groups per wave (D <=
// 4096 over 16 waves; with more, the 16 tokens' x strips outgrow the LDS).
constexpr bool gu16_fits(int64_t m, int64_t gpw) { return m >= 5 && m <= 16 && gpw <= 2; }

int launch_gu16(int64_t gpw, int64_t tiles, hipStream_t s, const DiagArgs& a) {
    if (a.ksplit != 1 || !gu16_fits(a.m, gpw))
        return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: %d tokens at %lld groups per wave", a.m, (long long)gpw);
    if (!a.xsum || !aligned(a.xsum, 4))
        return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: no place for the block sums of h");
    // two tiles per block where one per block would take more than one round
    const bool two = tiles > device_cu_count();
    const unsigned grid = static_cast<unsigned>(two ? (tiles + 1) / 2 : tiles);
#define TQ_GU16(G, P)                                                                                             \
    k_decode_gu16<G, P><<<grid, kBlock, 0, s>>>(a.x, a.m, a.pt, a.st, a.n, a.k, a.hout, a.xsum, a.tok0, a.mtot, \
                                                a.rows_group, a.yz, a.yz_n)
    if (gpw <= 1) {
        if (two)
            TQ_GU16(1, 2);
        else
            TQ_GU16(1, 1);
    } else {
        if (two)
            TQ_GU16(2, 2);
        else
            TQ_GU16(2, 1);
    }
#undef TQ_GU16
    return check_launch("tq_mlp_w4g128_decode");
}

template <int kEpi>
int launch_diag_r(int kr, int64_t gpw, int64_t tiles, hipStream_t s, const DiagArgs& a) {
    if (kr == 1) return launch_diag_m<1, kEpi>(gpw, tiles, s, a);
    if (kr == 2) return launch_diag_m<2, kEpi>(gpw, tiles, s, a);
    return launch_diag_m<4, kEpi>(gpw, tiles, s, a);
}

template <int kR>
int launch_mfma(int64_t gpw, int64_t tiles, hipStream_t s, const uint16_t* x, int m, const uint8_t* pt,
                const uint16_t* st, const float* b, int64_t n, int64_t k, float* y) {
    const unsigned grid = static_cast<unsigned>(tiles);
    // runs of up to 2 groups: x staged through LDS (the 16 token rows fit)
    if (gpw <= 1)
        k_decode_tiled_mfma_sx<kR, 1><<<grid, kBlock, 0, s>>>(x, m, pt, st, b, n, k, y);
    else if (gpw <= 2)
        k_decode_tiled_mfma_sx<kR, 2><<<grid, kBlock, 0, s>>>(x, m, pt, st, b, n, k, y);
    else
        k_decode_tiled_mfma<kR, 4><<<grid, kBlock, 0, s>>>(x, m, pt, st, b, n, k, y);
    return check_launch("tq_gemv_w4g128_tiled");
}

// The decode FFN's down projection for 5-16 tokens in one launch (2t <= 32 rows
// of h, 32-row tiles, K split in two onto a zeroed y); gpw is the groups per
// wave of one K half over the kernel's 8 waves.
template <int kSets>
void launch_fold32_sets(int64_t gpw, const dim3& grid, hipStream_t s, const uint16_t* h, int rows,
                        const uint8_t* pt, const uint16_t* st, int64_t n, int64_t k, float* y) {
    constexpr unsigned kThreads = kFoldWaves * 64;
#define TQ_FOLD(G) k_decode_fold32<G, kSets><<<grid, kThreads, 0, s>>>(h, rows, pt, st, n, k, y)
    switch (gpw) {
        case 1: TQ_FOLD(1); break;
        case 2: TQ_FOLD(2); break;
        case 3: TQ_FOLD(3); break;
        case 4: TQ_FOLD(4); break;
        case 5: TQ_FOLD(5); break;
        case 6: TQ_FOLD(6); break;
        case 7: TQ_FOLD(7); break;
        default: TQ_FOLD(8); break;
    }
#undef TQ_FOLD
}

int launch_fold32(int64_t gpw, int64_t tiles, hipStream_t s, const uint16_t* h, int rows, const uint8_t* pt,
                  const uint16_t* st, int64_t n, int64_t k, float* y) {
    if (gpw < 1 || gpw > 8 || rows > 32 || rows % 2 != 0)
        return fail(TQ_EINVAL, "tq_mlp_w4g128_decode: %d rows of h at %lld groups per wave", rows, (long long)gpw);
    const dim3 grid(static_cast<unsigned>(tiles), 2u);
    if (rows <= 16)
        launch_fold32_sets<1>(gpw, grid, s, h, rows, pt, st, n, k, y);
    else
        launch_fold32_sets<2>(gpw, grid, s, h, rows, pt, st, n, k, y);
    return check_launch("tq_mlp_w4g128_decode");
}

// Repack into the tiled layout through LDS: a block takes 2048 / T chunks (rounded
// down to whole groups of 4; about 32 KB in all) of each of one tile's T rows, reading the rows contiguously (consecutive
// threads, consecutive chunks of a row), and writes them back in tile order
// (consecutive threads, consecutive rows of a chunk).  The source of tile row r
// of tile t is row t*half + r % half of `pa` (r < half) or `pb`: half = T for a
// single weight, 32 for the FFN's gate (pa) / up (pb) interleave in 64-row tiles.
// The block also copies the f16 scales of its chunks' groups.  Rows at or past
// `nrows` are zero.
constexpr int kRepackItems = 2048;  // 16-byte chunks per block

__global__ __launch_bounds__(256) void k_repack_lds(const uint8_t* __restrict__ pa, const uint16_t* __restrict__ sa,
                                                    const uint8_t* __restrict__ pb, const uint16_t* __restrict__ sb,
                                                    int64_t nrows, int64_t k, int tile_rows, int half,
                                                    int64_t cblocks, uint8_t* __restrict__ pt,
                                                    uint16_t* __restrict__ st) {
    __shared__ __attribute__((aligned(16))) uint8_t buf[kRepackItems * 16 + 64 * 16];
    const int T = tile_rows, cpb = (kRepackItems / T) & ~3;  // whole groups of 4 chunks
    const int row_b = cpb * 16 + 16;  // padded LDS row: consecutive rows 4 banks apart
    const int64_t C = k >> 5, G = k >> 7;
    const int64_t t = blockIdx.x / cblocks, c0 = (blockIdx.x % cblocks) * cpb;
    const int nc = static_cast<int>(min<int64_t>(cpb, C - c0));
    // the f16 scales of the block's groups (4 chunks each): s_t[(t*G + g)*T + r]
    for (int it = threadIdx.x; it < (nc >> 2) * T; it += 256) {
        const int gg = it / T, r = it - gg * T;
        const int64_t g = (c0 >> 2) + gg, row = t * half + r % half;
        st[(t * G + g) * T + r] = row < nrows ? (r < half ? sa : sb)[row * G + g] : uint16_t(0);
    }
    for (int it = threadIdx.x; it < T * cpb; it += 256) {
        const int r = it / cpb, cc = it - r * cpb;
        const int64_t row = t * half + r % half;
        const uint8_t* src = r < half ? pa : pb;
        u32x4 v = u32x4{0u, 0u, 0u, 0u};
        if (cc < nc && row < nrows) v = *reinterpret_cast<const u32x4*>(src + row * (k >> 1) + (c0 + cc) * 16);
        *reinterpret_cast<u32x4*>(buf + r * row_b + cc * 16) = v;
    }
    __syncthreads();
    for (int it = threadIdx.x; it < nc * T; it += 256) {
        const int cc = it / T, r = it - cc * T;
        reinterpret_cast<u32x4*>(pt)[(t * C + c0 + cc) * T + r] =
            *reinterpret_cast<const u32x4*>(buf + r * row_b + cc * 16);
    }
}

int launch_repack(const uint8_t* pa, const uint16_t* sa, const uint8_t* pb, const uint16_t* sb, int64_t nrows,
                  int64_t k, int tile_rows, int half, int64_t tiles, uint8_t* pt, uint16_t* st, hipStream_t s,
                  const char* what) {
    const int64_t C = k >> 5, cpb = (kRepackItems / tile_rows) & ~3, cblocks = (C + cpb - 1) / cpb;
    if (tiles * cblocks >= (int64_t(1) << 31)) return fail(TQ_EINVAL, "%s: problem too large", what);
    k_repack_lds<<<static_cast<unsigned>(tiles * cblocks), 256, 0, s>>>(pa, sa, pb, sb, nrows, k, tile_rows, half,
                                                                        cblocks, pt, st);
    return check_launch(what);
}

template <int kM, int kCPW>
void launch_tiled(int64_t tiles, hipStream_t s, const uint16_t* x, const uint8_t* pt, const uint16_t* st,
                  const float* b, int64_t n, int64_t k, int T, float* y) {
    k_decode_tiled<kM, kCPW><<<static_cast<unsigned>(tiles), kBlock, 0, s>>>(x, pt, st, b, n, k, T, y);
}

// dispatch on chunks-per-wave (kCPW in {1, 2, 4, 8, 16, 32}: a wave may own a
// few chunks past K, which are clamped and masked)
template <int kM>
void dispatch_tiled(int64_t cpw, int64_t tiles, hipStream_t s, const uint16_t* x, const uint8_t* pt,
                    const uint16_t* st, const float* b, int64_t n, int64_t k, int T, float* y) {
    if (cpw <= 1) launch_tiled<kM, 1>(tiles, s, x, pt, st, b, n, k, T, y);
    else if (cpw <= 2) launch_tiled<kM, 2>(tiles, s, x, pt, st, b, n, k, T, y);
    else if (cpw <= 4) launch_tiled<kM, 4>(tiles, s, x, pt, st, b, n, k, T, y);
    else if (cpw <= 8) launch_tiled<kM, 8>(tiles, s, x, pt, st, b, n, k, T, y);
    else if (cpw <= 16) launch_tiled<kM, 16>(tiles, s, x, pt, st, b, n, k, T, y);
    else launch_tiled<kM, 32>(tiles, s, x, pt, st, b, n, k, T, y);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int64_t tq_w4g128_tile_rows(int64_t n) {
    // about one tile per CU, in {16, 32, 64} rows (the MFMA kernel's row groups)
    if (n <= 0) return 16;
    const int64_t cus = device_cu_count();
    const int64_t t = (n + cus - 1) / cus;
    return t <= 16 ? 16 : (t <= 32 ? 32 : 64);
}

int tq_repack_w4g128_tiled(const uint8_t* packed, const uint16_t* s_f16, int64_t n, int64_t k,
                           int64_t tile_rows, uint8_t* packed_t, uint16_t* s_t, tq_stream_t stream) {
    TQ_REQUIRE(n >= 0 && k >= 0, "tq_repack_w4g128_tiled: negative shape");
    TQ_REQUIRE(k % 128 == 0, "tq_repack_w4g128_tiled: K=%lld is not a multiple of 128", (long long)k);
    TQ_REQUIRE(tile_rows >= 8 && tile_rows <= 64 && tile_rows % 8 == 0,
               "tq_repack_w4g128_tiled: tile_rows=%lld must be a multiple of 8 in [8, 64]", (long long)tile_rows);
    if (n == 0 || k == 0) return TQ_OK;
    TQ_REQUIRE(packed && s_f16 && packed_t && s_t, "tq_repack_w4g128_tiled: null pointer");
    TQ_REQUIRE(aligned(packed, 16) && aligned(packed_t, 16) && aligned(s_f16, 2) && aligned(s_t, 2),
               "tq_repack_w4g128_tiled: misaligned pointer (packed buffers need 16 B)");
    const int64_t tiles = (n + tile_rows - 1) / tile_rows;
    return launch_repack(packed, s_f16, packed, s_f16, n, k, static_cast<int>(tile_rows), static_cast<int>(tile_rows),
                         tiles, packed_t, s_t, as_hip(stream), "tq_repack_w4g128_tiled");
}

int tq_gemv_w4g128_tiled(const uint16_t* x_bf16, int64_t m, const uint8_t* packed_t, const uint16_t* s_t,
                         const float* bias, int64_t n, int64_t k, int64_t tile_rows, float* y,
                         tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemv_w4g128_tiled: negative shape");
    TQ_REQUIRE(m <= 16, "tq_gemv_w4g128_tiled: M=%lld > 16", (long long)m);
    TQ_REQUIRE(k % 128 == 0, "tq_gemv_w4g128_tiled: K=%lld is not a multiple of 128", (long long)k);
    TQ_REQUIRE(tile_rows >= 8 && tile_rows <= 64 && tile_rows % 8 == 0,
               "tq_gemv_w4g128_tiled: tile_rows=%lld must be a multiple of 8 in [8, 64]", (long long)tile_rows);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(k > 0 && y, "tq_gemv_w4g128_tiled: K=0 or null y");
    const int64_t cpw = ((k >> 5) + kWaves - 1) / kWaves;
    TQ_REQUIRE(cpw <= kMaxCPW, "tq_gemv_w4g128_tiled: K=%lld > %d", (long long)k, kMaxCPW * kWaves * 32);
    TQ_REQUIRE(x_bf16 && packed_t && s_t, "tq_gemv_w4g128_tiled: null pointer");
    TQ_REQUIRE(aligned(x_bf16, 8) && aligned(packed_t, 16) && aligned(s_t, 2) && (!bias || aligned(bias, 4)) &&
                   aligned(y, 4),
               "tq_gemv_w4g128_tiled: misaligned pointer (packed_t needs 16 B, x 8 B)");
    const int64_t tiles = (n + tile_rows - 1) / tile_rows;
    const int T = static_cast<int>(tile_rows);
    const hipStream_t st = as_hip(stream);
    const int kr = T == 16 ? 1 : (T == 32 ? 2 : (T == 64 ? 4 : 0));
    const int64_t gpw = ((k >> 7) + kWaves - 1) / kWaves;
    // 1-4 tokens: the diagonal MFMA kernel (3-4 tokens on 64-row tiles: 7.6-8.0
    // against 8.4 us for the kernel below at 14336 x 4096)
    if (kr && aligned(x_bf16, 8) && aligned(s_t, 8) && m <= 4) {
        const DiagArgs a{x_bf16, static_cast<int>(m), packed_t, s_t, bias, n, k, y, nullptr, 0, 0};
        return launch_diag_r<kEpiPlain>(kr, gpw, tiles, st, a);
    }
    // 5..16 tokens: the MFMA kernel where the tile is 16, 32 or 64 rows, the 16 waves'
    // K runs are at most 4 groups (K <= 8192) and x rows are 16-byte aligned
    if (m >= 3 && kr && gpw <= 4 && aligned(x_bf16, 16) && aligned(s_t, 8)) {
        const int mi = static_cast<int>(m);
        if (kr == 1) return launch_mfma<1>(gpw, tiles, st, x_bf16, mi, packed_t, s_t, bias, n, k, y);
        if (kr == 2) return launch_mfma<2>(gpw, tiles, st, x_bf16, mi, packed_t, s_t, bias, n, k, y);
        return launch_mfma<4>(gpw, tiles, st, x_bf16, mi, packed_t, s_t, bias, n, k, y);
    }
    for (int64_t m0 = 0; m0 < m; m0 += kMaxTok) {
        const int64_t mm = (m - m0) < kMaxTok ? (m - m0) : kMaxTok;
        const uint16_t* xp = x_bf16 + m0 * k;
        float* yp = y + m0 * n;
        if (mm == 1) dispatch_tiled<1>(cpw, tiles, st, xp, packed_t, s_t, bias, n, k, T, yp);
        else if (mm == 2) dispatch_tiled<2>(cpw, tiles, st, xp, packed_t, s_t, bias, n, k, T, yp);
        else if (mm == 3) dispatch_tiled<3>(cpw, tiles, st, xp, packed_t, s_t, bias, n, k, T, yp);
        else dispatch_tiled<4>(cpw, tiles, st, xp, packed_t, s_t, bias, n, k, T, yp);
        const int rc = check_launch("tq_gemv_w4g128_tiled");
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

int64_t tq_mlp_w4g128_decode_workspace_bytes(int64_t m, int64_t d, int64_t f) {
    if (m < 0 || d < 0 || f < 0) return -1;
    return tq::mlp_h_bytes(m, f) + tq::round_up256(2 * m * ((f + 31) / 32) * 4);
}

int tq_repack_w4g128_gate_up_tiled(const uint8_t* gate_packed, const uint16_t* gate_s, const uint8_t* up_packed,
                                   const uint16_t* up_s, int64_t f, int64_t d, uint8_t* packed_t, uint16_t* s_t,
                                   tq_stream_t stream) {
    TQ_REQUIRE(f >= 0 && d >= 0, "tq_repack_w4g128_gate_up_tiled: negative shape");
    TQ_REQUIRE(d % 128 == 0, "tq_repack_w4g128_gate_up_tiled: D=%lld is not a multiple of 128", (long long)d);
    if (f == 0 || d == 0) return TQ_OK;
    TQ_REQUIRE(gate_packed && gate_s && up_packed && up_s && packed_t && s_t,
               "tq_repack_w4g128_gate_up_tiled: null pointer");
    TQ_REQUIRE(aligned(gate_packed, 16) && aligned(up_packed, 16) && aligned(packed_t, 16) && aligned(gate_s, 2) &&
                   aligned(up_s, 2) && aligned(s_t, 2),
               "tq_repack_w4g128_gate_up_tiled: misaligned pointer (packed buffers need 16 B)");
    const int64_t tiles = (f + 31) / 32;
    return launch_repack(gate_packed, gate_s, up_packed, up_s, f, d, 64, 32, tiles, packed_t, s_t, as_hip(stream),
                         "tq_repack_w4g128_gate_up_tiled");
}

}  // extern "C"

namespace tq {
namespace {

// Scratch of the allocation-free decode FFN: the bf16 hi and lo rows of h and
// their 32-column sums for 16 tokens at F = 16384 (the largest decode shape).  One copy per device, held
// until the process ends; host code reaches it only through the address that
// hipGetSymbolAddress returns for the current device.
constexpr int64_t kMlpDecodeScratch = mlp_h_bytes(16, 16384) + round_up256(2 * 16 * (16384 / 32) * 4);
static_assert(kMlpDecodeScratch == TQ_MLP_DECODE_SCRATCH_BYTES, "tq.h states the scratch size");
__device__ __align__(256) uint8_t scratch[kMlpDecodeScratch];

std::atomic<void*> g_scratch_ptr[64];
std::mutex g_scratch_mu;

// Device address of `scratch` on the current device (resolved once per device).
int scratch_address(const char* fn, void** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(TQ_EHIP, "%s: hipGetDevice failed", fn);
    void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
    if (!p) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
        if (!p) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || !p)
                return fail(TQ_EHIP, "%s: hipGetSymbolAddress(scratch) on device %d: %s", fn, dev,
                            hipGetErrorString(e));
            g_scratch_ptr[dev].store(p, std::memory_order_release);
        }
    }
    *out = p;
    return TQ_OK;
}

// Checks and launches of the decode FFN.  With `use_scratch` set, h goes to the
// current device's scratch array (resolved after the arguments are checked)
// and `workspace` is ignored.
int mlp_decode(const char* fn, const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f, const uint8_t* gate_up_t,
               const uint16_t* gate_up_s_t, const uint8_t* down_t, const uint16_t* down_s_t,
               int64_t down_tile_rows, void* workspace, int64_t workspace_bytes, bool use_scratch, float* y,
               tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && d >= 0 && f >= 0, "%s: negative shape", fn);
    TQ_REQUIRE(m <= 16, "%s: M=%lld > 16", fn, (long long)m);
    TQ_REQUIRE(d % 128 == 0 && f % 128 == 0, "%s: D=%lld and F=%lld must be multiples of 128", fn,
               (long long)d, (long long)f);
    TQ_REQUIRE(d <= kMaxCPW * kWaves * 32 && f <= kMaxCPW * kWaves * 32,
               "%s: D=%lld or F=%lld > %d", fn, (long long)d, (long long)f, kMaxCPW * kWaves * 32);
    TQ_REQUIRE(down_tile_rows == 16 || down_tile_rows == 32 || down_tile_rows == 64,
               "%s: down tile_rows=%lld must be 16, 32 or 64", fn, (long long)down_tile_rows);
    if (m == 0 || d == 0) return TQ_OK;
    TQ_REQUIRE(f > 0, "%s: F=0", fn);
    TQ_REQUIRE(x_bf16 && gate_up_t && gate_up_s_t && down_t && down_s_t && (workspace || use_scratch) && y,
               "%s: null pointer", fn);
    const int64_t need = tq_mlp_w4g128_decode_workspace_bytes(m, d, f);
    if (use_scratch) {
        TQ_REQUIRE(need <= kMlpDecodeScratch, "%s: M=%lld, F=%lld need %lld bytes of scratch, more than its %lld",
                   fn, (long long)m, (long long)f, (long long)need, (long long)kMlpDecodeScratch);
        if (int rc = scratch_address(fn, &workspace)) return rc;
        workspace_bytes = kMlpDecodeScratch;
    }
    TQ_REQUIRE(workspace_bytes >= need, "%s: workspace of %lld bytes, %lld needed", fn,
               (long long)workspace_bytes, (long long)need);
    TQ_REQUIRE(aligned(x_bf16, 8) && aligned(gate_up_t, 16) && aligned(down_t, 16) && aligned(gate_up_s_t, 8) &&
                   aligned(down_s_t, 8) && aligned(workspace, 16) && aligned(y, 4),
               "%s: misaligned pointer", fn);
    const hipStream_t st = as_hip(stream);
    uint16_t* h = static_cast<uint16_t*>(workspace);
    float* hsum = reinterpret_cast<float*>(static_cast<uint8_t*>(workspace) + mlp_h_bytes(m, f));
    const int64_t fb = f >> 5;  // 32-column blocks of a row of h
    const int mi = static_cast<int>(m);
    // gate + up with SiLU * up, 4 tokens per launch, into the hi/lo rows of h
    const int kr = down_tile_rows == 16 ? 1 : (down_tile_rows == 32 ? 2 : 4);
    // Quads: one down launch per four tokens (their 2t hi/lo rows as MFMA
    // columns), K split over two blocks per tile so that the x rows fit the LDS;
    // the gate/up launch zeroes y for the two halves.  Taken for 3-4 tokens on
    // 16-row down tiles and for 1-4 tokens on 32-row tiles, whose 128 tiles x 2 K
    // halves fill 256 CUs in one round at D = 4096.
    const bool block = (kr == 1 && (mi == 3 || mi == 4)) || kr == 2;
    // 5-16 tokens on 32-row down tiles: all 2m <= 32 rows of h in one down launch
    // (k_decode_fold32: one set of 16 MFMA columns up to 8 tokens, two beyond),
    // the down weights read once
    const bool one_down = kr == 2 && mi >= 5;
    const int group = one_down ? 16 : (block ? 4 : 2);  // tokens per MlpRows group
    const int64_t gu_tiles = (f + 31) / 32, gu_gpw = ((d >> 7) + kWaves - 1) / kWaves;
    // 5-16 tokens: one launch of the 16x16x32 kernel where its x strips fit the LDS
    const bool gu16 = gu16_fits(mi, gu_gpw);
    if (gu16) {
        DiagArgs a{x_bf16, mi, gate_up_t, gate_up_s_t, nullptr, 2 * f, d, nullptr, h, 0, mi};
        a.rows_group = group;
        a.xsum = hsum;
        if (block) {
            a.yz = y;
            a.yz_n = m * d;
        }
        const int rc = launch_gu16(gu_gpw, gu_tiles, st, a);
        if (rc != TQ_OK) return rc;
    }
    for (int j0 = 0; j0 < mi && !gu16; j0 += 4) {
        const int mm = mi - j0 < 4 ? mi - j0 : 4;
        DiagArgs a{x_bf16 + j0 * d, mm, gate_up_t, gate_up_s_t, nullptr, 2 * f, d, nullptr, h, j0, mi};
        a.rows_group = group;
        a.xsum = hsum;
        if (block && j0 == 0) {
            a.yz = y;
            a.yz_n = m * d;
        }
        const int rc = launch_diag_m<4, kEpiGateUp>(gu_gpw, gu_tiles, st, a);
        if (rc != TQ_OK) return rc;
    }
    const int64_t dn_tiles = (d + down_tile_rows - 1) / down_tile_rows, dn_gpw = ((f >> 7) + kWaves - 1) / kWaves;
    const int64_t gpw2 = (((f >> 7) + 1) / 2 + kWaves - 1) / kWaves;  // of a K half
    if (one_down) {
        const int64_t gpw8 = (((f >> 7) + 1) / 2 + kFoldWaves - 1) / kFoldWaves;  // of a K half, 8 waves
        return launch_fold32(gpw8, dn_tiles, st, h, 2 * mi, down_t, down_s_t, d, f, y);
    }
    if (block) {
        for (int c = 0; 4 * c < mi; ++c) {
            const int t = mi - 4 * c < 4 ? mi - 4 * c : 4;
            DiagArgs a{h + 8 * c * f, 2 * t, down_t, down_s_t, nullptr, d, f, y + 4 * c * d, nullptr, 0, 0};
            a.ksplit = 2;
            a.xsum = hsum + 8 * c * fb;
            const int rc = launch_diag_r<kEpiFold>(kr, gpw2, dn_tiles, st, a);
            if (rc != TQ_OK) return rc;
        }
        return TQ_OK;
    }
    // down, one launch per token pair: its hi and lo rows in, their sum out
    for (int c = 0; 2 * c < mi; ++c) {
        const int t = mi - 2 * c < 2 ? mi - 2 * c : 2;
        DiagArgs a{h + 4 * c * f, 2 * t, down_t, down_s_t, nullptr, d, f, y + 2 * c * d, nullptr, 0, 0};
        a.xsum = hsum + 4 * c * fb;
        const int rc = launch_diag_r<kEpiFold>(kr, dn_gpw, dn_tiles, st, a);
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

}  // namespace
}  // namespace tq

extern "C" {

int tq_mlp_w4g128_decode(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f, const uint8_t* gate_up_t,
                         const uint16_t* gate_up_s_t, const uint8_t* down_t, const uint16_t* down_s_t,
                         int64_t down_tile_rows, void* workspace, int64_t workspace_bytes, float* y,
                         tq_stream_t stream) {
    return mlp_decode("tq_mlp_w4g128_decode", x_bf16, m, d, f, gate_up_t, gate_up_s_t, down_t, down_s_t,
                      down_tile_rows, workspace, workspace_bytes, false, y, stream);
}

int tq_mlp_w4g128_decode_noalloc(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                                 const uint8_t* gate_up_t, const uint16_t* gate_up_s_t, const uint8_t* down_t,
                                 const uint16_t* down_s_t, int64_t down_tile_rows, float* y, tq_stream_t stream) {
    // nothing is allocated: h goes to this device's scratch array
    return mlp_decode("tq_mlp_w4g128_decode_noalloc", x_bf16, m, d, f, gate_up_t, gate_up_s_t, down_t, down_s_t,
                      down_tile_rows, nullptr, 0, true, y, stream);
}

}  // extern "C"
