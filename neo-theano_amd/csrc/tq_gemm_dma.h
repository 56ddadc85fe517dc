// tq_gemm_dma.h -- the W8A8 GEMM's DMA kernel (k_gemm_w8a8_dma) and the pieces
// the FP8 GEMM shares with it: tile order, DMA plan, stage ring, fragment reads
// and epilogue.  Included by tq_gemm.hip (the library) and by the bench
// library's phase-timing entry point, which instantiates the same kernel with
// timestamps (kTimed).  See tq_gemm.hip for the design.
#pragma once

#include "tq_internal.h"

namespace tq {
namespace {

// ------------------------------------------------------------- DMA kernel

constexpr int kDmaBM = 128, kDmaBN = 256, kDmaBK = 128;
constexpr int kDmaW = kDmaBN * kDmaBK;         // weight bytes per stage
constexpr int kDmaStage = kDmaW + kDmaBM * kDmaBK;
constexpr int kDmaEpiRow = 128 * 4 + 16;       // int32 row of a wave's 64 x 128 tile, padded
constexpr int kDmaGroupM = 8;                  // m tiles per tile group (XCD locality)

// 16 bytes per lane from `g` into LDS at (l + 16 * lane).  The kernel tracks
// completion itself with explicit vmcnt waits (vmcnt retires in order, so any
// wait the compiler adds for its own loads stays conservative).
__device__ __forceinline__ void dma16(const int8_t* g, int8_t* l) { lds_dma16(g, lds_addr(l)); }

// XOR swizzle of the 16-byte chunk index of a 128-byte LDS row
__device__ __forceinline__ int dma_swz(int row) { return (row >> 1) & 7; }

struct DmaFrags {
    i32x4 w[4], a[2];
};

struct DmaCtx {
    const int8_t* src[12];  // per-lane DMA sources at k = 0 (8 weight, 4 activation)
    int wave, wm, wn, lane;
};

__device__ __forceinline__ int8_t* dma_dst(const DmaCtx& c, int8_t* st, int t) {
    return t < 8 ? st + (8 * c.wave + t) * 1024 : st + kDmaW + (4 * c.wave + (t - 8)) * 1024;
}

// MFMA operand of row `row`, K chunk kc (32 bytes): lane l supplies 16 bytes,
// chunk 2 kc + l / 32 of the row.
__device__ __forceinline__ i32x4 dma_frag(const int8_t* base, int row, int kc, int lane) {
    const int c = 2 * kc + (lane >> 5);
    return *reinterpret_cast<const i32x4*>(base + row * kDmaBK + ((c ^ dma_swz(row)) << 4));
}

#define TQ_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// 8 MFMAs on `cur`; meanwhile read the 6 fragments of chunk nkc of stage buffer
// `nst` into `nxt` and issue DMAs t0..t0+2 of the stage at byte offset k0 into `dst`.
__device__ __forceinline__ void dma_step(const DmaFrags& cur, DmaFrags& nxt, const int8_t* nst, int nkc,
                                         const DmaCtx& c, int t0, int k0, int8_t* dst, i32x16 (&acc)[4][2]) {
    const int lr = c.lane & 31;
#define TQ_MF(i, j) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(cur.w[i], cur.a[j], acc[i][j], 0, 0, 0)
    TQ_MF(0, 0);
    nxt.w[0] = dma_frag(nst, c.wn * 128 + 0 * 32 + lr, nkc, c.lane);
    TQ_SCHED_FENCE();
    TQ_MF(0, 1);
    nxt.w[1] = dma_frag(nst, c.wn * 128 + 1 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0] + k0, dma_dst(c, dst, t0));
    TQ_SCHED_FENCE();
    TQ_MF(1, 0);
    nxt.w[2] = dma_frag(nst, c.wn * 128 + 2 * 32 + lr, nkc, c.lane);
    TQ_SCHED_FENCE();
    TQ_MF(1, 1);
    nxt.w[3] = dma_frag(nst, c.wn * 128 + 3 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 1] + k0, dma_dst(c, dst, t0 + 1));
    TQ_SCHED_FENCE();
    TQ_MF(2, 0);
    nxt.a[0] = dma_frag(nst + kDmaW, c.wm * 64 + 0 * 32 + lr, nkc, c.lane);
    TQ_SCHED_FENCE();
    TQ_MF(2, 1);
    nxt.a[1] = dma_frag(nst + kDmaW, c.wm * 64 + 1 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 2] + k0, dma_dst(c, dst, t0 + 2));
    TQ_SCHED_FENCE();
    TQ_MF(3, 0);
    TQ_SCHED_FENCE();
    TQ_MF(3, 1);
    TQ_SCHED_FENCE();
#undef TQ_MF
}

// Tile of this block: blocks are dealt to the 8 XCDs round robin; give each XCD
// a contiguous range of tiles, ordered in groups of kDmaGroupM m tiles (n
// fastest), so that the blocks sharing an L2 share operand rows.
__device__ __forceinline__ void dma_tile(int tiles_m, int tiles_n, int* m0, int* n0) {
    const int T = tiles_m * tiles_n;
    const int b = blockIdx.x;
    const int L = (T % 8 == 0) ? (b % 8) * (T / 8) + b / 8 : b;
    const int gm = tiles_m % kDmaGroupM == 0 ? kDmaGroupM : 1;
    const int grp = L / (gm * tiles_n);
    const int tm = grp * gm + (L % gm), tn = (L / gm) % tiles_n;
    *n0 = tn * kDmaBN;
    *m0 = tm * kDmaBM;
}

// DMA t moves rows 8 s .. 8 s + 7 of the stage (s = slot): lane -> row s*8 + lane/8,
// global chunk (lane % 8) ^ swz(row) lands in LDS chunk lane % 8.  Rows past the
// matrix edge re-read its last row (those outputs are never stored).
__device__ __forceinline__ void dma_sources(DmaCtx& c, const int8_t* qa, const int8_t* qw, int m0, int n0, int m,
                                            int n, int k) {
#pragma unroll
    for (int t = 0; t < 12; ++t) {
        const bool isw = t < 8;
        const int slot = isw ? 8 * c.wave + t : 4 * c.wave + (t - 8);
        const int row = slot * 8 + (c.lane >> 3);
        const int koff = ((c.lane & 7) ^ dma_swz(row)) * 16;
        const int r = isw ? min(n0 + row, n - 1) : min(m0 + row, m - 1);
        c.src[t] = (isw ? qw : qa) + static_cast<int64_t>(r) * k + koff;
    }
}

__device__ __forceinline__ float acc_value(int32_t bits, i32x16) { return static_cast<float>(bits); }
__device__ __forceinline__ float acc_value(int32_t bits, f32x16) { return __builtin_bit_cast(float, bits); }

// Epilogue: lane holds D[n = 8 (r / 4) + 4 (l / 32) + r % 4][m = l % 32] of each
// 32 x 32 tile.  Each wave writes its 64 x 128 tile (4-byte words) to LDS as
// rows, reads it back with lane = 4 consecutive n and stores 512-byte row
// segments: y = f32(acc) * sa[m] * sw[n] (+ b[n]); acc_out gets the raw int32
// accumulators of the integer kernel.
template <class Acc>
__device__ __forceinline__ void dma_epilogue(const Acc (&acc)[4][2], const DmaCtx& c, int8_t* lds, int m0, int n0,
                                             int m, int n, const float* __restrict__ sa,
                                             const float* __restrict__ sw, const float* __restrict__ bias,
                                             int32_t* __restrict__ acc_out, float* __restrict__ y) {
    const int lane = c.lane;
    int8_t* ep = lds + c.wave * (64 * kDmaEpiRow);
    const int lr = lane & 31, lh = lane >> 5;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            // the whole vector is bit-cast: a bit cast of a single element of a
            // vector lvalue here compiled to a copy of element 0 for every element
            const i32x16 bits = __builtin_bit_cast(i32x16, acc[i][j]);
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const i32x4 v = i32x4{bits[4 * g], bits[4 * g + 1], bits[4 * g + 2], bits[4 * g + 3]};
                *reinterpret_cast<i32x4*>(ep + (j * 32 + lr) * kDmaEpiRow + (i * 32 + 8 * g + 4 * lh) * 4) = v;
            }
        }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int nb = n0 + c.wn * 128 + 4 * lr;
    const bool nval = nb < n;
    f32x4 swv = f32x4{0.f, 0.f, 0.f, 0.f}, bv = f32x4{0.f, 0.f, 0.f, 0.f};
    if (nval) {
        swv = *reinterpret_cast<const f32x4*>(sw + nb);
        if (bias) bv = *reinterpret_cast<const f32x4*>(bias + nb);
    }
    const float sa_lane = sa[min(m0 + c.wm * 64 + lane, m - 1)];
#pragma unroll 4
    for (int rr = 0; rr < 64; rr += 2) {
        const int row = rr + lh;
        const int mm = m0 + c.wm * 64 + row;
        const i32x4 v = *reinterpret_cast<const i32x4*>(ep + row * kDmaEpiRow + lr * 16);
        const float s_row = __shfl(sa_lane, row, kWave);
        if (nval && mm < m) {
            if (acc_out) *reinterpret_cast<i32x4*>(acc_out + static_cast<int64_t>(mm) * n + nb) = v;
            f32x4 o;
            o.x = fmaf(acc_value(v.x, Acc{}) * s_row, swv.x, bv.x);
            o.y = fmaf(acc_value(v.y, Acc{}) * s_row, swv.y, bv.y);
            o.z = fmaf(acc_value(v.z, Acc{}) * s_row, swv.z, bv.z);
            o.w = fmaf(acc_value(v.w, Acc{}) * s_row, swv.w, bv.w);
            __builtin_nontemporal_store(o, reinterpret_cast<f32x4*>(y + static_cast<int64_t>(mm) * n + nb));
        }
    }
}

// kTimed (the bench library's instantiation only): lane 0 of every wave writes
// the real-time clock (100 MHz) at its start, once the first stage has landed,
// after the K loop and after the epilogue's stores, and the wave's hardware
// id, to ts[(block * 4 + wave) * 6 ..].
template <bool kTimed = false>
__global__ __launch_bounds__(256, 1) void k_gemm_w8a8_dma(const int8_t* __restrict__ qa,
                                                          const float* __restrict__ sa,
                                                          const int8_t* __restrict__ qw,
                                                          const float* __restrict__ sw,
                                                          const float* __restrict__ bias, int m, int n,
                                                          int k, int32_t* __restrict__ acc_out,
                                                          float* __restrict__ y, int tiles_m,
                                                          int tiles_n, uint64_t* __restrict__ ts = nullptr) {
    uint64_t t[4] = {0, 0, 0, 0};
    if constexpr (kTimed) t[0] = __builtin_amdgcn_s_memrealtime();
    __shared__ __attribute__((aligned(1024))) int8_t lds[3 * kDmaStage];
    DmaCtx c;
    const int tid = threadIdx.x;
    c.lane = tid & 63;
    c.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    c.wm = c.wave & 1;
    c.wn = c.wave >> 1;
    const int lane = c.lane;
    int m0, n0;
    dma_tile(tiles_m, tiles_n, &m0, &n0);
    dma_sources(c, qa, qw, m0, n0, m, n, k);

    i32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = i32x16{};

    const int ks_n = k / kDmaBK;
    const int k_last = (ks_n - 1) * kDmaBK;  // stages past the end re-read the last one (never used)
#pragma unroll
    for (int t = 0; t < 12; ++t) dma16(c.src[t], dma_dst(c, lds, t));
#pragma unroll
    for (int t = 0; t < 12; ++t) dma16(c.src[t] + min(kDmaBK, k_last), dma_dst(c, lds + kDmaStage, t));
    asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
    if constexpr (kTimed) t[1] = __builtin_amdgcn_s_memrealtime();
    DmaFrags f0, f1;
    {
        const int lr = lane & 31;
#pragma unroll
        for (int i = 0; i < 4; ++i) f0.w[i] = dma_frag(lds, c.wn * 128 + i * 32 + lr, 0, lane);
#pragma unroll
        for (int j = 0; j < 2; ++j) f0.a[j] = dma_frag(lds + kDmaW, c.wm * 64 + j * 32 + lr, 0, lane);
    }
    // Ring: stage ks in buffer ks % 3; its 4 K chunks run as 4 steps.  The DMAs
    // of stage ks + 2 (into the buffer stage ks - 1 used) are spread over the 4
    // steps: 9 before the barrier, 3 after.
    int rd = 0;
    for (int ks = 0; ks < ks_n; ++ks) {
        int8_t* st = lds + rd * kDmaStage;
        const int nrd = rd == 2 ? 0 : rd + 1;
        const int drd = nrd == 2 ? 0 : nrd + 1;
        int8_t* dst = lds + drd * kDmaStage;
        const int k0 = min((ks + 2) * kDmaBK, k_last);
        dma_step(f0, f1, st, 1, c, 0, k0, dst, acc);
        dma_step(f1, f0, st, 2, c, 3, k0, dst, acc);
        dma_step(f0, f1, st, 3, c, 6, k0, dst, acc);
        // Stage ks + 1 has landed once at most the 9 DMAs just issued are
        // outstanding; after the barrier every wave is past its reads of buffer rd.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(9)\n\ts_barrier" ::: "memory");
        dma_step(f1, f0, lds + nrd * kDmaStage, 0, c, 9, k0, dst, acc);
        rd = nrd;
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if constexpr (kTimed) t[2] = __builtin_amdgcn_s_memrealtime();
    dma_epilogue(acc, c, lds, m0, n0, m, n, sa, sw, bias, acc_out, y);
    if constexpr (kTimed) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stores have left the wave
        t[3] = __builtin_amdgcn_s_memrealtime();
        uint32_t hwid;
        asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hwid));
        if (lane == 0) {
            uint64_t* o = ts + (static_cast<int64_t>(blockIdx.x) * 4 + c.wave) * 6;
            for (int i = 0; i < 4; ++i) o[i] = t[i];
            o[4] = hwid;
            o[5] = 0;
        }
    }
}

}  // namespace
}  // namespace tq
