// tq_ffn.hip -- the quantized Llama-style FFN block (INT4 g128 gate/up/down,
// bf16 activations) on gfx950 bf16 MFMA with an LDS-DMA pipeline.
//
// Reference composition: Linear::forward (crates/theano-nn/src/linear.rs:111-121)
// over dequantized weights, SiLU (crates/theano-nn/src/activation.rs:66-79,
// x * 1/(1+exp(-x))) and Tensor::mul, all in f64; here f32 accumulation.
//
// Three launches:
//   prep    x -> xp (x with each 4-block (a,b,c,d) stored (a,c,b,d), the order
//           the weight unpack produces) and X[g][m] = -192 * sum of group g of
//           row m, stored as three bf16 planes (hi, mid, lo) whose sum is the
//           f32 value; zeroes y (the down launch adds two K halves into it).
//   gate/up one block per 128 (or 64) rows x 128 columns of h; h = SiLU(x Wg^T) * (x Wu^T)
//           is written as bf16 hi + lo planes (hi + lo keeps ~2^-17 of h) in
//           the xp order, with the same -192 * group-sum planes for the down
//           projection (a block's 128 columns are one of its groups).
//   down    one block per 64 rows x 256 (or 64) columns and half of K; the two halves
//           are added into the zeroed y with float atomics (two addends onto
//           zero: the sum does not depend on their order).
//
// Weights: a nibble q (two's complement) becomes bf16 8*(24+q): q+8 (xor 8) is
// put in the top four mantissa bits of bf16 128.  An MFMA over a 128-long group
// therefore gives 8 * (sum q x + 24 sum x); the -192 * group-sum planes, fed
// through one extra MFMA per group (planes as A, ones as B), cancel the offset.
// The offset 24 (not the 136 of a low-mantissa nibble) keeps the running sums
// of a group within a few times their final size, so the f32 rounding inside
// the MFMA chain stays small.
//
// Group scales: one accumulator per output tile runs across groups in units of
// the current group's scale; at a group change it is multiplied by
// s_prev / s_cur (16 multiplies per tile, no second accumulator), and the
// epilogue multiplies by s_last / 8.
//
// Pipeline (per block, 8 waves): stages of one group (128 k) are copied
// global -> LDS by global_load_lds_dwordx4 (activations, weights; 16-byte
// chunks XOR-swizzled against bank conflicts) and global_load_lds_dword
// (scales: one dword per weight row holds the scales of groups 2j and 2j+1;
// X planes) into a ring of three stage buffers, two stages ahead of the
// MFMAs.  Per stage: one barrier, issued after the last fragment reads of the
// stage, after which the next stage's operands are read while the last MFMAs
// of the stage run.  MFMA: v_mfma_f32_32x32x16_bf16, A = activations (m), B =
// unpacked weights (n), so each lane's 16 outputs share one n (one scale).
#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kOffset = 192.0f;  // 8 * 24: weight operand 8 * (24 + q)
constexpr float kUnit = 0.125f;    // 1 / 8

// 64 lanes x 16 bytes -> LDS [la, la + 1024)
__device__ __forceinline__ void dma16(const int8_t* g, uint32_t la) { lds_dma16(g, la); }
// active lanes x 4 bytes -> LDS la + 4 * lane
__device__ __forceinline__ void dma4(const int8_t* g, uint32_t la) { lds_dma4(g, la); }
#define TQ_FENCE() __builtin_amdgcn_sched_barrier(0)

// Makes a value opaque to the optimizer: keeps the prologue's LDS reads of the
// first stage from being merged with the loop's reads of the next stage into
// one read at the loop head (which would expose its latency every stage).
template <typename V>
__device__ __forceinline__ void opaque(V& v) {
    asm volatile("" : "+v"(v));
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t to_bf16(float f) {
    return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(f)));
}
__device__ __forceinline__ float from_bf16(uint32_t b) { return __uint_as_float(b << 16); }

// f32 -> bf16 planes (hi, mid, lo), hi + mid + lo == v: dwords (hi | mid << 16, lo)
__device__ __forceinline__ uint2 split3(float v) {
    const uint32_t h = to_bf16(v);
    const float r1 = v - from_bf16(h);
    const uint32_t md = to_bf16(r1);
    const uint32_t lo = to_bf16(r1 - from_bf16(md));
    return make_uint2(h | (md << 16), lo);
}

// Packed dword of 8 nibbles (k..k+7, low nibble first) -> bf16 8 * (24 + q) in
// the slot order (k, k+2), (k+1, k+3), (k+4, k+6), (k+5, k+7).  The byte
// ((q + 8) << 3) is ((w ^ 0x88888888) << 3 or >> 1) & 0x78 per byte, written as
// one shift and one three-input bit operation.
__device__ __forceinline__ u32x4 unpack8(uint32_t w) {
    const uint32_t lo = ((w << 3) & 0x78787878u) ^ 0x40404040u;
    const uint32_t hi = ((w >> 1) & 0x78787878u) ^ 0x40404040u;
    u32x4 a;
    a.x = __builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u);
    a.y = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);
    a.z = __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u);
    a.w = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);
    return a;
}

__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// 16 lanes per (row, group): 8 values each.  Also zeroes y [M, ny] when given
// (grid-stride, 16 bytes per step).
__global__ __launch_bounds__(256) void k_ffn_prep(const uint16_t* __restrict__ x, int64_t m, int64_t d, int64_t mpad,
                                                  uint16_t* __restrict__ xp, uint32_t* __restrict__ xs,
                                                  float* __restrict__ yzero, int64_t ny) {
    if (yzero) {
        const int64_t n4 = m * ny / 4, stride = static_cast<int64_t>(gridDim.x) * 256;
        for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n4; i += stride)
            reinterpret_cast<f32x4*>(yzero)[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const int64_t G = d >> 7;
    const int64_t item = static_cast<int64_t>(blockIdx.x) * 16 + (threadIdx.x >> 4);
    if (item >= m * G) return;
    const int64_t row = item / G, g = item - row * G;
    const int l = threadIdx.x & 15;
    const int64_t off = row * d + g * 128 + 8 * l;
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + off);
    float s = (bf16_lo(v.x) + bf16_hi(v.x)) + (bf16_lo(v.y) + bf16_hi(v.y)) + (bf16_lo(v.z) + bf16_hi(v.z)) +
              (bf16_lo(v.w) + bf16_hi(v.w));
    s = lane_group_sum<16>(s);  // a group's 16 lanes are one DPP row
    u32x4 o;
    o.x = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);
    o.y = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);
    o.z = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);
    o.w = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);
    *reinterpret_cast<u32x4*>(xp + off) = o;
    if (l == 0) *reinterpret_cast<uint2*>(xs + (g * mpad + row) * 2) = split3(-kOffset * s);
}

struct FfnArgs {
    const uint16_t* a0;  // activation plane(s) [M, K] bf16 in xp order
    const uint16_t* a1;
    const uint32_t* xs;  // -192 * group sums of the activations, planes [K/128][mpad][2]
    const uint8_t* w0;   // INT4 g128 [N, K/2]: gate (gate/up) or down
    const uint16_t* s0;  // f16 [N, K/128]
    const uint8_t* w1;   // up (gate/up only)
    const uint16_t* s1;
    int64_t m, n, k, mpad;
    int tiles_m, tiles_n;
    float* y;        // down / Linear: f32 [M, N], zeroed when K is split
    const float* bias;  // Linear: f32 [N] or null
    uint16_t* h_hi;  // gate/up: h planes [M, N] bf16 in xp order
    uint16_t* h_lo;
    uint32_t* hs;    // gate/up: -192 * group sums of h, planes [N/128][mpad][2]
};

// Block: kWavesM x kWavesN waves; a wave owns kWM 32-row tiles and kTN
// 32-column tiles of each of kMats weight matrices; kPlanes activation planes.
template <int kWavesM, int kWavesN, int kWM, int kTN, int kMats, int kPlanes>
struct FfnCfg {
    static constexpr int kWaves = kWavesM * kWavesN, kThreads = 64 * kWaves;
    static constexpr int BM = kWavesM * 32 * kWM, BN = kWavesN * 32 * kTN, WRows = kMats * BN;
    static constexpr int kTiles = kMats * kTN;
    // stage layout: activations (kPlanes x BM rows x 256 B), weights (WRows x 64 B),
    // scale dwords (WRows x 4 B), X planes (BM x 8 B, padded)
    static constexpr int ABytes = kPlanes * BM * 256, WBytes = WRows * 64;
    static constexpr int SOff = ABytes + WBytes, SBytes = WRows * 4;
    static constexpr int SD = SBytes / 4 + BM * 2;  // dwords of scales and X planes
    static constexpr int kSmallLanes = SD <= 32 * kWaves ? 32 : 64;  // one 4-byte DMA per wave
    static_assert(SD <= 64 * kWaves && (SBytes / 4) % kSmallLanes == 0, "scale / X DMAs");
    static constexpr int XOff = SOff + SBytes, XBytes = kWaves * kSmallLanes * 4 - SBytes;
    static constexpr int Stage = XOff + XBytes;
    static constexpr int NA = ABytes / 1024, NW = WBytes / 1024;
    static constexpr int kBig = (NA + NW) / kWaves, kD = kBig + 1;  // DMAs per wave per stage
    static_assert((NA + NW) % kWaves == 0, "uniform DMA count per wave");
    static_assert(3 * Stage <= 160 * 1024, "three stages in LDS");
    // DMA j of a stage is issued after the MFMAs of step dma_step(j) (steps 0..6)
    static constexpr int dma_step(int j) { return (j * 7) / kD; }
};

template <int kWavesM, int kWavesN, int kWM, int kTN, int kMats, int kPlanes, int kSplit>
__global__ __launch_bounds__(64 * kWavesM * kWavesN, 1) void k_ffn(FfnArgs p) {
    using C = FfnCfg<kWavesM, kWavesN, kWM, kTN, kMats, kPlanes>;
    constexpr int BM = C::BM, BN = C::BN, kTiles = C::kTiles, kD = C::kD, kBig = C::kBig;
    constexpr bool kGateUp = kMats == 2;
    __shared__ __attribute__((aligned(1024))) int8_t lds[3 * C::Stage];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % kWavesM, wn = wave / kWavesM;
    const int l32 = lane & 31, lh = lane >> 5;
    // consecutive blocks go to different XCDs: give each XCD a contiguous run of
    // tiles (row tiles fastest) so that blocks sharing weight rows share an L2
    const int T = p.tiles_m * p.tiles_n * kSplit, b = blockIdx.x;
    const int L = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int tm = L % p.tiles_m, ks = (L / p.tiles_m) % kSplit, tn_blk = L / (p.tiles_m * kSplit);
    const int64_t m0 = static_cast<int64_t>(tm) * BM, n0 = static_cast<int64_t>(tn_blk) * BN;
    const int G = static_cast<int>(p.k >> 7);                         // groups of K (scale row length)
    const int g0 = ks * G / kSplit, ng = (ks + 1) * G / kSplit - g0;  // this block's groups
    const int64_t rowA = p.k * 2, rowW = p.k >> 1;

    // DMA plan: per DMA j a per-lane source at group 0, bytes per group, shift of
    // the group index (scale dwords hold two groups) and the LDS offset in a stage
    const int8_t* dsrc[kD];
    int64_t dstride[kD];
    int dshift[kD];
    uint32_t doff[kD];
#pragma unroll
    for (int j = 0; j < kD; ++j) {
        if (j < kBig) {
            const int t = wave * kBig + j;
            doff[j] = t * 1024;
            dshift[j] = 0;
            if (t < C::NA) {  // 4 activation rows, chunk c of row r at slot c ^ (r & 15)
                const int pl = t / (BM / 4), r = (t % (BM / 4)) * 4 + (lane >> 4);
                const int c = (lane & 15) ^ (r & 15);
                const int64_t row = min<int64_t>(m0 + r, p.m - 1);
                dsrc[j] = reinterpret_cast<const int8_t*>(pl ? p.a1 : p.a0) + row * rowA + c * 16;
                dstride[j] = 256;
            } else {  // 16 weight rows, chunk c of row r at slot c ^ ((r >> 2) & 3)
                const int wr = (t - C::NA) * 16 + (lane >> 2);
                const int c = (lane & 3) ^ ((wr >> 2) & 3);
                const int mat = wr / BN;
                const int64_t nrow = n0 + wr % BN;
                dsrc[j] = reinterpret_cast<const int8_t*>(mat ? p.w1 : p.w0) + nrow * rowW + c * 16;
                dstride[j] = 64;
            }
        } else {
            doff[j] = C::SOff + wave * C::kSmallLanes * 4;
            const int q = wave * C::kSmallLanes + min(lane, C::kSmallLanes - 1);  // dword of the area
            if (wave * C::kSmallLanes < C::WRows) {
                const int mat = q / BN;
                const int64_t nrow = n0 + q % BN;
                dsrc[j] = reinterpret_cast<const int8_t*>((mat ? p.s1 : p.s0) + nrow * G);
                dstride[j] = 4;
                dshift[j] = 1;
            } else {
                dsrc[j] = reinterpret_cast<const int8_t*>(p.xs + m0 * 2 + min(q - C::WRows, BM * 2 - 1));
                dstride[j] = p.mpad * 8;
                dshift[j] = 0;
            }
        }
    }
    const uint32_t lds0 = lds_addr(lds);
    // stages past the last group re-read the last group into a buffer nobody reads
    auto dma = [&](int j, int s, int buf) {
        const int g = g0 + min(s, ng - 1);
        const int8_t* src = dsrc[j] + static_cast<int64_t>(g >> dshift[j]) * dstride[j];
        const uint32_t la = lds0 + buf * C::Stage + doff[j];
        if (j < kBig)
            dma16(src, la);
        else if (C::kSmallLanes == 64 || lane < C::kSmallLanes)
            dma4(src, la);
    };

    struct Ops {
        uint32_t sraw[kTiles];  // f16 scale of the lane's column, per B tile
        uint2 xa[kWM];          // X planes of the lane's row, per A tile
        u32x4 wf[kTiles][2];    // the lane's 32 bytes of its weight row
    };
    auto load_ops = [&](int buf, int s, Ops& o) {
        const int8_t* st = lds + buf * C::Stage;
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const int mat = t / kTN, tn = t % kTN;
            const int wr = mat * BN + wn * 32 * kTN + tn * 32 + l32;
            o.sraw[t] = *reinterpret_cast<const uint16_t*>(st + C::SOff + wr * 4 + ((g0 + s) & 1) * 2);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int c = (2 * j + lh) ^ ((wr >> 2) & 3);
                o.wf[t][j] = *reinterpret_cast<const u32x4*>(st + C::ABytes + wr * 64 + c * 16);
            }
        }
#pragma unroll
        for (int i = 0; i < kWM; ++i) {
            const int r = wm * 32 * kWM + i * 32 + l32;
            o.xa[i] = *reinterpret_cast<const uint2*>(st + C::XOff + r * 8);
        }
    };
    // A fragments of step `step` (k 16 step .. +15): lane reads chunk 8 (step/4) + 4 lh + step%4
    auto load_a = [&](int buf, int step, u32x4 (&a)[kWM][kPlanes]) {
        const int8_t* st = lds + buf * C::Stage;
        const int cA = 8 * (step >> 2) + 4 * lh + (step & 3);
#pragma unroll
        for (int i = 0; i < kWM; ++i) {
            const int r = wm * 32 * kWM + i * 32 + l32;
#pragma unroll
            for (int pl = 0; pl < kPlanes; ++pl)
                a[i][pl] = *reinterpret_cast<const u32x4*>(st + (pl * BM + r) * 256 + ((cA ^ (r & 15)) << 4));
        }
    };

    // ones for the X planes (k 0..2 of the lanes 0..31)
    const u32x4 bone = lh == 0 ? u32x4{0x3F803F80u, 0x00003F80u, 0u, 0u} : u32x4{0u, 0u, 0u, 0u};
    f32x16 dg[kWM][kTiles];
#pragma unroll
    for (int i = 0; i < kWM; ++i)
#pragma unroll
        for (int t = 0; t < kTiles; ++t) dg[i][t] = f32x16{};
    float sprev[kTiles];

    // prologue: stages 0 and 1 in flight, wait for stage 0
#pragma unroll
    for (int j = 0; j < kD; ++j) dma(j, 0, 0);
#pragma unroll
    for (int j = 0; j < kD; ++j) dma(j, 1, 1);
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kD) : "memory");
    Ops nx;
    u32x4 an[kWM][kPlanes];
    load_ops(0, 0, nx);
    load_a(0, 0, an);
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        opaque(nx.sraw[t]);
        opaque(nx.wf[t][0]);
        opaque(nx.wf[t][1]);
    }
#pragma unroll
    for (int i = 0; i < kWM; ++i) {
        opaque(nx.xa[i].x);
        opaque(nx.xa[i].y);
#pragma unroll
        for (int pl = 0; pl < kPlanes; ++pl) opaque(an[i][pl]);
    }
#pragma unroll
    for (int t = 0; t < kTiles; ++t) sprev[t] = __half2float(__ushort_as_half(static_cast<uint16_t>(nx.sraw[t])));

    int rd = 0;
    for (int s = 0; s < ng; ++s) {
        const int nrd = rd == 2 ? 0 : rd + 1;
        const int drd = nrd == 2 ? 0 : nrd + 1;  // buffer of stage s + 2 (= stage s - 1)
        const Ops cur = nx;
        float ratio[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const float sc = __half2float(__ushort_as_half(static_cast<uint16_t>(cur.sraw[t])));
            ratio[t] = sprev[t] * __builtin_amdgcn_rcpf(sc);
            sprev[t] = sc;
        }
        u32x4 a[kWM][kPlanes];
#pragma unroll
        for (int i = 0; i < kWM; ++i)
#pragma unroll
            for (int pl = 0; pl < kPlanes; ++pl) a[i][pl] = an[i][pl];
#pragma unroll
        for (int step = 0; step < 8; ++step) {
            const int j = step >> 2, d = step & 3;
            u32x4 bw[kTiles];
#pragma unroll
            for (int t = 0; t < kTiles; ++t) bw[t] = unpack8(cur.wf[t][j][d]);
            if (step < 7) {
                load_a(rd, step + 1, an);
            } else {
                // stage s + 1 landed for every wave and every wave is done reading stage s
                TQ_FENCE();
                asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kD) : "memory");
                TQ_FENCE();
                load_ops(nrd, s + 1, nx);
                load_a(nrd, 0, an);
            }
#pragma unroll
            for (int i = 0; i < kWM; ++i) {
                if (step == 0) {
                    const u32x4 xa = lh == 0 ? u32x4{cur.xa[i].x, cur.xa[i].y, 0u, 0u} : u32x4{0u, 0u, 0u, 0u};
#pragma unroll
                    for (int t = 0; t < kTiles; ++t) {
#pragma unroll
                        for (int e = 0; e < 16; ++e) dg[i][t][e] *= ratio[t];
                        dg[i][t] = mfma(xa, bone, dg[i][t]);
                    }
                }
#pragma unroll
                for (int t = 0; t < kTiles; ++t)
#pragma unroll
                    for (int pl = 0; pl < kPlanes; ++pl) dg[i][t] = mfma(a[i][pl], bw[t], dg[i][t]);
            }
#pragma unroll
            for (int jj = 0; jj < kD; ++jj)
                if (C::dma_step(jj) == step) dma(jj, s + 2, drd);
            if (step < 7) {
#pragma unroll
                for (int i = 0; i < kWM; ++i)
#pragma unroll
                    for (int pl = 0; pl < kPlanes; ++pl) a[i][pl] = an[i][pl];
            }
        }
        rd = nrd;
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // lane holds D[m = 8 (e/4) + 4 lh + e % 4][n = l32] of each 32 x 32 tile
    if constexpr (!kGateUp) {
#pragma unroll
        for (int i = 0; i < kWM; ++i)
#pragma unroll
            for (int t = 0; t < kTiles; ++t) {
                const int64_t nn = n0 + wn * 32 * kTN + t * 32 + l32;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int64_t mm = m0 + wm * 32 * kWM + i * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
                    if (mm < p.m) {
                        const float v = (kUnit * sprev[t]) * dg[i][t][e] + (p.bias && ks == 0 ? p.bias[nn] : 0.0f);
                        if constexpr (kSplit == 1)
                            p.y[mm * p.n + nn] = v;
                        else
                            unsafeAtomicAdd(p.y + mm * p.n + nn, v);
                    }
                }
            }
    } else {
        static_assert(BN == 128, "a block's h columns are one group of the down projection");
        constexpr int kHRow = BN + 4;
        float* hsm = reinterpret_cast<float*>(lds);
#pragma unroll
        for (int i = 0; i < kWM; ++i)
#pragma unroll
            for (int tn = 0; tn < kTN; ++tn)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float g = (kUnit * sprev[tn]) * dg[i][tn][e];
                    const float u = (kUnit * sprev[kTN + tn]) * dg[i][kTN + tn][e];
                    const float hv = g * (1.0f / (1.0f + __expf(-g))) * u;
                    const int r = wm * 32 * kWM + i * 32 + 8 * (e >> 2) + 4 * lh + (e & 3);
                    hsm[r * kHRow + wn * 32 * kTN + tn * 32 + l32] = hv;
                }
        __syncthreads();
        constexpr int kTPR = C::kThreads / BM;  // threads per h row
        constexpr int kCols = BN / kTPR;
        const int r = tid / kTPR, q = tid % kTPR;
        const int64_t mm = m0 + r;
        const int64_t o = mm * p.n + n0 + q * kCols;
        float sum = 0.0f;
#pragma unroll
        for (int c8 = 0; c8 < kCols / 8; ++c8) {
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(hsm + r * kHRow + q * kCols + c8 * 8);
            const f32x4 v1 = *reinterpret_cast<const f32x4*>(hsm + r * kHRow + q * kCols + c8 * 8 + 4);
            const float hv[8] = {v0.x, v0.z, v0.y, v0.w, v1.x, v1.z, v1.y, v1.w};  // xp order
            uint32_t hb[8], lb[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                hb[e] = to_bf16(hv[e]);
                lb[e] = to_bf16(hv[e] - from_bf16(hb[e]));
                sum += from_bf16(hb[e]) + from_bf16(lb[e]);
            }
            if (mm < p.m) {
                *reinterpret_cast<u32x4*>(p.h_hi + o + c8 * 8) =
                    u32x4{hb[0] | (hb[1] << 16), hb[2] | (hb[3] << 16), hb[4] | (hb[5] << 16), hb[6] | (hb[7] << 16)};
                *reinterpret_cast<u32x4*>(p.h_lo + o + c8 * 8) =
                    u32x4{lb[0] | (lb[1] << 16), lb[2] | (lb[3] << 16), lb[4] | (lb[5] << 16), lb[6] | (lb[7] << 16)};
            }
        }
        sum = lane_group_sum<kTPR>(sum);
        if (q == 0 && mm < p.m) *reinterpret_cast<uint2*>(p.hs + (tn_blk * p.mpad + mm) * 2) = split3(-kOffset * sum);
    }
}

// gate/up: 2 x 4 waves of 64 rows x (32 gate + 32 up) columns -> 128 x 128 h per block
constexpr int kGuWM = 2, kGuWN = 4, kGuTM = 2, kGuTN = 1;
using GuCfg = FfnCfg<kGuWM, kGuWN, kGuTM, kGuTN, 2, 1>;
// down: 2 x 4 waves of 32 rows x 64 columns on two h planes -> 64 x 256 y per block, K in two halves
constexpr int kDnWM = 2, kDnWN = 4, kDnTM = 1, kDnTN = 2, kDnSplit = 2;
using DnCfg = FfnCfg<kDnWM, kDnWN, kDnTM, kDnTN, 1, 2>;

// prefill Linear: 2 x 4 waves of 64 rows x 64 columns -> 128 x 256 y per block
constexpr int kLnWM = 2, kLnWN = 4, kLnTM = 2, kLnTN = 2;
using LinCfg = FfnCfg<kLnWM, kLnWN, kLnTM, kLnTN, 1, 1>;

// Narrow tiles for mid-size M, where the tiles above leave most CUs idle or run
// padding rows (at M = 64 the 128-row gate/up tiles are half padding and the
// down projection has 32 blocks): gate/up 64 x 128 h (2 x 4 waves of 32 rows x
// (32 gate + 32 up)), down 64 x 64 y (2 x 2 waves of 32 x 32 on the two planes,
// K in two halves), Linear 64 x 128 y (2 x 4 waves of 32 x 32).
using GuSCfg = FfnCfg<2, 4, 1, 1, 2, 1>;
using DnSCfg = FfnCfg<2, 2, 1, 1, 1, 2>;
using LinSCfg = FfnCfg<2, 4, 1, 1, 1, 1>;

// Relative time of a launch: rounds of blocks over the CUs times the MFMA work of
// one block (BM x BN x groups of K) times the time per unit of work of the tile
// set, in thousandths of the wide tiles' (narrow tiles move more bytes per MFMA:
// per block-round at D = 4096, F = N = 14336, gate/up 64-row tiles take 1.25x,
// the 64 x 64 down tiles 1.4x and the 64 x 128 Linear tiles ~1.25x the wide
// tiles' time per MFMA).  The tile set with the smaller figure runs; ties keep
// the wide tiles.
constexpr int64_t kWideCost = 1000, kNarrowGuCost = 1250, kNarrowDnCost = 1400, kNarrowLinCost = 1250;
int64_t launch_cost(int64_t blocks, int64_t bm, int64_t bn, int64_t groups, int64_t per_unit) {
    const int64_t cus = device_cu_count();
    return (blocks + cus - 1) / cus * bm * bn * groups * per_unit;
}

struct FfnWorkspace {
    int64_t mpad, xp, xs, hh, hl, hs, bytes;  // byte offsets of the parts, total
};

int64_t align256(int64_t v) { return (v + 255) / 256 * 256; }

FfnWorkspace ffn_workspace(int64_t m, int64_t d, int64_t f) {
    FfnWorkspace w{};
    w.mpad = (m + 127) / 128 * 128;
    w.xp = 0;
    w.xs = align256(w.xp + m * d * 2);
    w.hh = align256(w.xs + (d / 128) * w.mpad * 8);
    w.hl = align256(w.hh + m * f * 2);
    w.hs = align256(w.hl + m * f * 2);
    w.bytes = align256(w.hs + (f / 128) * w.mpad * 8);
    return w;
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int64_t tq_mlp_w4g128_workspace_bytes(int64_t m, int64_t d, int64_t f) {
    if (m <= 0 || d <= 0 || f <= 0) return 0;
    // the shape-general path keeps h as f32 [M, F] in the same buffer
    const int64_t fast = ffn_workspace(m, d, f).bytes, general = m * f * 4;
    return fast > general ? fast : general;
}

int tq_mlp_w4g128(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f, const uint8_t* gate_packed,
                  const uint16_t* gate_s, const uint8_t* up_packed, const uint16_t* up_s,
                  const uint8_t* down_packed, const uint16_t* down_s, void* workspace, int64_t workspace_bytes,
                  float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && d >= 0 && f >= 0, "tq_mlp_w4g128: negative shape");
    TQ_REQUIRE(d % 128 == 0 && f % 128 == 0,
               "tq_mlp_w4g128: D=%lld and F=%lld must be multiples of 128", (long long)d, (long long)f);
    if (m == 0 || d == 0) return TQ_OK;
    TQ_REQUIRE(f > 0, "tq_mlp_w4g128: F=0");
    TQ_REQUIRE(x_bf16 && gate_packed && gate_s && up_packed && up_s && down_packed && down_s && workspace && y,
               "tq_mlp_w4g128: null pointer");
    const int64_t need = tq_mlp_w4g128_workspace_bytes(m, d, f);
    TQ_REQUIRE(workspace_bytes >= need, "tq_mlp_w4g128: workspace of %lld bytes, %lld needed",
               (long long)workspace_bytes, (long long)need);
    TQ_REQUIRE(aligned(x_bf16, 16) && aligned(gate_packed, 16) && aligned(up_packed, 16) &&
                   aligned(down_packed, 16) && aligned(workspace, 16) && aligned(y, 16),
               "tq_mlp_w4g128: misaligned pointer (16 B required)");
    TQ_REQUIRE(aligned(gate_s, 2) && aligned(up_s, 2) && aligned(down_s, 2), "tq_mlp_w4g128: misaligned scales");
    const hipStream_t st = as_hip(stream);
    // the pipelined kernels read scale pairs as dwords (an even number of groups,
    // 4-byte aligned scales) and tile the output columns by 128 (gate/up) and 256 (down)
    const bool fast = d % 256 == 0 && f % 256 == 0 && aligned(gate_s, 4) && aligned(up_s, 4) && aligned(down_s, 4) &&
                      aligned(workspace, 256);
    if (!fast)
        return launch_mlp_w4g128_general(x_bf16, m, d, f, gate_packed, gate_s, up_packed, up_s, down_packed, down_s,
                                         static_cast<float*>(workspace), y, st);

    const FfnWorkspace w = ffn_workspace(m, d, f);
    uint8_t* base = static_cast<uint8_t*>(workspace);
    uint16_t* xp = reinterpret_cast<uint16_t*>(base + w.xp);
    uint32_t* xs = reinterpret_cast<uint32_t*>(base + w.xs);
    uint16_t* hh = reinterpret_cast<uint16_t*>(base + w.hh);
    uint16_t* hl = reinterpret_cast<uint16_t*>(base + w.hl);
    uint32_t* hs = reinterpret_cast<uint32_t*>(base + w.hs);

    const int64_t items = m * (d / 128);
    TQ_REQUIRE((items + 15) / 16 < (int64_t(1) << 31), "tq_mlp_w4g128: problem too large");
    // wide or narrow tiles per launch, whichever leaves less work on the busiest CU
    static_assert(GuCfg::BN == GuSCfg::BN && DnCfg::BM == DnSCfg::BM, "the tile sets share these sides");
    const int64_t gu_tm = (m + GuCfg::BM - 1) / GuCfg::BM, gus_tm = (m + GuSCfg::BM - 1) / GuSCfg::BM;
    const int64_t gu_tn = f / GuCfg::BN, dn_tm = (m + DnCfg::BM - 1) / DnCfg::BM;
    const bool gu_narrow = launch_cost(gus_tm * gu_tn, GuSCfg::BM, GuSCfg::BN, d / 128, kNarrowGuCost) <
                           launch_cost(gu_tm * gu_tn, GuCfg::BM, GuCfg::BN, d / 128, kWideCost);
    const bool dn_narrow =
        launch_cost(dn_tm * (d / DnSCfg::BN) * kDnSplit, DnSCfg::BM, DnSCfg::BN, f / 256, kNarrowDnCost) <
        launch_cost(dn_tm * (d / DnCfg::BN) * kDnSplit, DnCfg::BM, DnCfg::BN, f / 256, kWideCost);
    const int64_t gu_tiles_m = gu_narrow ? gus_tm : gu_tm, gu_tiles = gu_tiles_m * gu_tn;
    const int64_t dn_tiles_n = d / (dn_narrow ? DnSCfg::BN : DnCfg::BN), dn_tiles = dn_tm * dn_tiles_n * kDnSplit;
    TQ_REQUIRE(gu_tiles < (int64_t(1) << 31) && dn_tiles < (int64_t(1) << 31), "tq_mlp_w4g128: problem too large");

    k_ffn_prep<<<static_cast<unsigned>((items + 15) / 16), 256, 0, st>>>(x_bf16, m, d, w.mpad, xp, xs, y, d);
    int rc = check_launch("tq_mlp_w4g128 (prep)");
    if (rc != TQ_OK) return rc;

    FfnArgs a{};
    a.a0 = xp;
    a.xs = xs;
    a.w0 = gate_packed;
    a.s0 = gate_s;
    a.w1 = up_packed;
    a.s1 = up_s;
    a.m = m;
    a.n = f;
    a.k = d;
    a.mpad = w.mpad;
    a.tiles_m = static_cast<int>(gu_tiles_m);
    a.tiles_n = static_cast<int>(gu_tn);
    a.h_hi = hh;
    a.h_lo = hl;
    a.hs = hs;
    if (gu_narrow)
        k_ffn<2, 4, 1, 1, 2, 1, 1><<<static_cast<unsigned>(gu_tiles), GuSCfg::kThreads, 0, st>>>(a);
    else
        k_ffn<kGuWM, kGuWN, kGuTM, kGuTN, 2, 1, 1><<<static_cast<unsigned>(gu_tiles), GuCfg::kThreads, 0, st>>>(a);
    rc = check_launch("tq_mlp_w4g128 (gate/up)");
    if (rc != TQ_OK) return rc;

    FfnArgs b{};
    b.a0 = hh;
    b.a1 = hl;
    b.xs = hs;
    b.w0 = down_packed;
    b.s0 = down_s;
    b.m = m;
    b.n = d;
    b.k = f;
    b.mpad = w.mpad;
    b.tiles_m = static_cast<int>(dn_tm);
    b.tiles_n = static_cast<int>(dn_tiles_n);
    b.y = y;
    if (dn_narrow)
        k_ffn<2, 2, 1, 1, 1, 2, kDnSplit><<<static_cast<unsigned>(dn_tiles), DnSCfg::kThreads, 0, st>>>(b);
    else
        k_ffn<kDnWM, kDnWN, kDnTM, kDnTN, 1, 2, kDnSplit>
            <<<static_cast<unsigned>(dn_tiles), DnCfg::kThreads, 0, st>>>(b);
    return check_launch("tq_mlp_w4g128 (down)");
}

// ---- prefill W4A16 Linear on the same kernels (one weight matrix, one plane) ----

int64_t tq_gemm_w4g128_bf16_workspace_bytes(int64_t m, int64_t k) {
    if (m <= 0 || k <= 0) return 0;
    const int64_t mpad = (m + 127) / 128 * 128;
    return align256(m * k * 2) + align256((k / 128) * mpad * 8);
}

int tq_gemm_w4g128_bf16_ws(const uint16_t* x_bf16, int64_t m, const uint8_t* packed, const uint16_t* s_f16,
                           const float* bias, int64_t n, int64_t k, void* workspace, int64_t workspace_bytes,
                           float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemm_w4g128_bf16_ws: negative shape");
    TQ_REQUIRE(k % 128 == 0, "tq_gemm_w4g128_bf16_ws: K=%lld is not a multiple of 128", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    const int64_t need = tq_gemm_w4g128_bf16_workspace_bytes(m, k);
    TQ_REQUIRE(k == 0 || (workspace && workspace_bytes >= need),
               "tq_gemm_w4g128_bf16_ws: workspace of %lld bytes, %lld needed", (long long)workspace_bytes,
               (long long)need);
    // the pipelined kernels: scale pairs as dwords (K % 256), 128- or 256-column
    // tiles, 16-byte vectors; anything else runs the workspace-free entry point
    const bool fast = k > 0 && k % 256 == 0 && n % LinSCfg::BN == 0 && x_bf16 && packed && s_f16 && y &&
                      aligned(x_bf16, 16) && aligned(packed, 16) && aligned(s_f16, 4) && aligned(y, 16) &&
                      (!bias || aligned(bias, 4)) && aligned(workspace, 256);
    if (!fast) return tq_gemm_w4g128_bf16(x_bf16, m, packed, s_f16, bias, n, k, y, stream);
    const hipStream_t st = as_hip(stream);
    const int64_t mpad = (m + 127) / 128 * 128;
    uint16_t* xp = static_cast<uint16_t*>(workspace);
    uint32_t* xs = reinterpret_cast<uint32_t*>(static_cast<uint8_t*>(workspace) + align256(m * k * 2));
    // K halves are added into y when the doubled grid still fits one round on the CUs
    // and each half keeps at least 8 groups (two addends onto zero: the sum does not
    // depend on their order).  Wide or narrow tiles, whichever leaves less work on
    // the busiest CU (wide ones need N % 256).
    auto plan = [&](int64_t bm, int64_t bn, int64_t per_unit, int64_t* tm, int64_t* tn, bool* split) {
        *tm = (m + bm - 1) / bm;
        *tn = n / bn;
        *split = 2 * *tm * *tn <= device_cu_count() && k / 128 >= 16;
        return launch_cost(*tm * *tn * (*split ? 2 : 1), bm, bn, k / 128 / (*split ? 2 : 1), per_unit);
    };
    int64_t tiles_m, tiles_n, wtm, wtn;
    bool split, wsplit;
    const int64_t narrow_cost = plan(LinSCfg::BM, LinSCfg::BN, kNarrowLinCost, &tiles_m, &tiles_n, &split);
    const bool narrow =
        n % LinCfg::BN != 0 || narrow_cost < plan(LinCfg::BM, LinCfg::BN, kWideCost, &wtm, &wtn, &wsplit);
    if (!narrow) {
        tiles_m = wtm;
        tiles_n = wtn;
        split = wsplit;
    }
    const int64_t items = m * (k / 128);
    TQ_REQUIRE((items + 15) / 16 < (int64_t(1) << 31) && tiles_m * tiles_n * 2 < (int64_t(1) << 31),
               "tq_gemm_w4g128_bf16_ws: problem too large");
    k_ffn_prep<<<static_cast<unsigned>((items + 15) / 16), 256, 0, st>>>(x_bf16, m, k, mpad, xp, xs,
                                                                       split ? y : nullptr, n);
    int rc = check_launch("tq_gemm_w4g128_bf16_ws (prep)");
    if (rc != TQ_OK) return rc;
    FfnArgs a{};
    a.a0 = xp;
    a.xs = xs;
    a.w0 = packed;
    a.s0 = s_f16;
    a.m = m;
    a.n = n;
    a.k = k;
    a.mpad = mpad;
    a.tiles_m = static_cast<int>(tiles_m);
    a.tiles_n = static_cast<int>(tiles_n);
    a.y = y;
    a.bias = bias;
    const unsigned blocks = static_cast<unsigned>(tiles_m * tiles_n * (split ? 2 : 1));
    if (narrow && split)
        k_ffn<2, 4, 1, 1, 1, 1, 2><<<blocks, LinSCfg::kThreads, 0, st>>>(a);
    else if (narrow)
        k_ffn<2, 4, 1, 1, 1, 1, 1><<<blocks, LinSCfg::kThreads, 0, st>>>(a);
    else if (split)
        k_ffn<kLnWM, kLnWN, kLnTM, kLnTN, 1, 1, 2><<<blocks, LinCfg::kThreads, 0, st>>>(a);
    else
        k_ffn<kLnWM, kLnWN, kLnTM, kLnTN, 1, 1, 1><<<blocks, LinCfg::kThreads, 0, st>>>(a);
    return check_launch("tq_gemm_w4g128_bf16_ws");
}

}  // extern "C"
