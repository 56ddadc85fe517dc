// tq_gemm.hip -- prefill-shaped W8A8 quantized Linear on gfx950 i8 MFMA.
//
//   acc[m, n] = sum_k qa[m, k] * qw[n, k]          (int32, exact)
//   y[m, n]   = f32(acc) * sa[m] * sw[n] (+ b[n])
//
// The reference value is Tensor::mm over the dequantized operands
// (crates/theano-core/src/tensor_ops.rs:379-410); over integral f64 codes that
// product is exact, so acc is bit-exact with it.
//
// Both operands are K-contiguous ("NT").  A dot product over K may visit K in
// any order as long as both operands use the same order, so each kernel picks
// the byte-to-lane assignment that suits its loads; integer accumulation makes
// the order invisible in the result.
//
// Two kernels:
//  * k_gemm_w8a8_dma (K % 128 == 0): one 256-thread block per 128 (m) x 256 (n)
//    tile.  K advances in 128-byte stages through a 3-deep LDS ring filled by
//    global_load_lds_dwordx4 (global -> LDS without registers; one instruction
//    moves 8 full 128-byte rows, XOR-swizzled by 16-byte chunk so the MFMA
//    fragment reads are bank-conflict free).  Four waves each own a 64 (m) x
//    128 (n) accumulator tile of v_mfma_i32_32x32x32_i8 (the i8 shape that
//    reaches full rate on gfx950; 16x16x64 issues at ~60%).  Every group of 8
//    MFMAs has the fragment reads of the next K chunk and 3 of the 12 DMA
//    instructions of the stage after next interleaved with it, so that neither
//    LDS latency nor a full memory queue idles the matrix core.  The epilogue
//    goes through LDS to write 512-byte row segments.
//  * k_gemm_w8a8 (any K % 16 == 0): 128 x 128 tiles of v_mfma_i32_16x16x64_i8
//    with register-staged LDS loads.
#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kBlock = 256;
constexpr int kTileN = 128;   // weight rows per block
constexpr int kTileM = 128;   // activation rows per block
constexpr int kTileK = 128;   // bytes of K per stage
constexpr int kLdsRow = kTileK + 16;

__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// Block tile order: an XCD receives every 8th block; renumber so that the 8
// blocks resident on one XCD at a time share weight tiles (column-major over m).
__device__ __forceinline__ void tile_of(int64_t bid, int64_t tiles_m, int64_t* tn, int64_t* tm) {
    *tn = bid / tiles_m;
    *tm = bid % tiles_m;
}

__global__ __launch_bounds__(kBlock, 2) void k_gemm_w8a8(const int8_t* __restrict__ qa,
                                                         const float* __restrict__ sa,
                                                         const int8_t* __restrict__ qw,
                                                         const float* __restrict__ sw,
                                                         const float* __restrict__ bias, int64_t m,
                                                         int64_t n, int64_t k,
                                                         int32_t* __restrict__ acc_out,
                                                         float* __restrict__ y) {
    __shared__ __attribute__((aligned(16))) int8_t lds_w[kTileN * kLdsRow];
    __shared__ __attribute__((aligned(16))) int8_t lds_a[kTileM * kLdsRow];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wn = wave >> 1, wm = wave & 1;  // 2 x 2 waves, each 64 n x 64 m
    const int64_t tiles_m = (m + kTileM - 1) / kTileM;
    int64_t tn, tm;
    tile_of(blockIdx.x, tiles_m, &tn, &tm);
    const int64_t n0 = tn * kTileN, m0 = tm * kTileM;

    // global -> register staging: thread t moves 16 B chunks (row t/8 + 32i, col 16*(t%8))
    const int ld_row = tid >> 3, ld_col = (tid & 7) * 16;
    i32x4 pw[4], pa[4];
    auto load_stage = [&](int64_t k0) {
        const bool kval = k0 + ld_col < k;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t rn = n0 + ld_row + 32 * i, rm = m0 + ld_row + 32 * i;
            pw[i] = (kval && rn < n) ? *reinterpret_cast<const i32x4*>(qw + rn * k + k0 + ld_col)
                                     : i32x4{0, 0, 0, 0};
            pa[i] = (kval && rm < m) ? *reinterpret_cast<const i32x4*>(qa + rm * k + k0 + ld_col)
                                     : i32x4{0, 0, 0, 0};
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            *reinterpret_cast<i32x4*>(lds_w + (ld_row + 32 * i) * kLdsRow + ld_col) = pw[i];
            *reinterpret_cast<i32x4*>(lds_a + (ld_row + 32 * i) * kLdsRow + ld_col) = pa[i];
        }
    };

    i32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    const int64_t ksteps = (k + kTileK - 1) / kTileK;
    load_stage(0);
    store_stage();
    __syncthreads();

    // MFMA operand rows: lane l reads row (l % 16) of a 16-row sub-tile, bytes
    // [16 * (l / 16), +16) of each 64-byte K step.
    const int op_row = lane & 15, op_k = (lane >> 4) * 16;
    for (int64_t ks = 0; ks < ksteps; ++ks) {
        if (ks + 1 < ksteps) load_stage((ks + 1) * kTileK);
#pragma unroll
        for (int kk = 0; kk < kTileK; kk += 64) {
            i32x4 a[4], b[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                a[i] = *reinterpret_cast<const i32x4*>(lds_w + (wn * 64 + i * 16 + op_row) * kLdsRow + kk + op_k);
                b[i] = *reinterpret_cast<const i32x4*>(lds_a + (wm * 64 + i * 16 + op_row) * kLdsRow + kk + op_k);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = mfma_i8(a[i], b[j], acc[i][j]);
        }
        __syncthreads();
        if (ks + 1 < ksteps) {
            store_stage();
            __syncthreads();
        }
    }

    // epilogue: lane holds D[n = 4*(l/16) + r][m = l % 16] of each 16x16 tile
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int64_t nb = n0 + wn * 64 + i * 16 + (lane >> 4) * 4;
        if (nb >= n) continue;
        const f32x4 swv = *reinterpret_cast<const f32x4*>(sw + nb);
        f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
        if (bias) bv = *reinterpret_cast<const f32x4*>(bias + nb);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int64_t mm = m0 + wm * 64 + j * 16 + (lane & 15);
            if (mm >= m) continue;
            const i32x4 c = acc[i][j];
            if (acc_out) *reinterpret_cast<i32x4*>(acc_out + mm * n + nb) = c;
            const float s_row = sa[mm];
            f32x4 o;
            o.x = fmaf(static_cast<float>(c.x) * s_row, swv.x, bv.x);
            o.y = fmaf(static_cast<float>(c.y) * s_row, swv.y, bv.y);
            o.z = fmaf(static_cast<float>(c.z) * s_row, swv.z, bv.z);
            o.w = fmaf(static_cast<float>(c.w) * s_row, swv.w, bv.w);
            *reinterpret_cast<f32x4*>(y + mm * n + nb) = o;
        }
    }
}


}  // namespace
}  // namespace tq

#include "tq_gemm_dma.h"

namespace tq {
namespace {

// ------------------------------------------------------------ FP8 (OCP e4m3)
// Same tiles, ring and epilogue as k_gemm_w8a8_dma, on v_mfma_f32_32x32x64_f8f6f4
// (A and B e4m3, f32 accumulators; the unscaled form of the f8f6f4 MFMA, which
// the builtin selects when both block scales are 0).  An MFMA consumes 64 bytes
// of K, so a 128-byte stage is 2 steps; each lane supplies 32 consecutive bytes
// of its row (16-byte chunks 4 kc + 2 (l / 32) and the next one).  Products of
// two e4m3 values are exact in f32; only the accumulation rounds.
struct Fp8Frags {
    i32x8 w[4], a[2];
};

__device__ __forceinline__ i32x8 fp8_frag(const int8_t* base, int row, int kc, int lane) {
    const int ch = 4 * kc + 2 * (lane >> 5);
    const int z = dma_swz(row);
    const int8_t* r = base + row * kDmaBK;
    const i32x4 lo = *reinterpret_cast<const i32x4*>(r + ((ch ^ z) << 4));
    const i32x4 hi = *reinterpret_cast<const i32x4*>(r + (((ch + 1) ^ z) << 4));
    return i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

__device__ __forceinline__ f32x16 mfma_fp8(i32x8 a, i32x8 b, f32x16 c) {
    // cbsz = blgp = 0: both operands FP8 E4M3; scales 0 select the unscaled MFMA
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// 8 MFMAs on `cur`; meanwhile read the 6 fragments of chunk nkc of stage buffer
// `nst` into `nxt` and issue DMAs t0..t0+5 of the stage at byte offset k0 into `dst`.
__device__ __forceinline__ void fp8_step(const Fp8Frags& cur, Fp8Frags& nxt, const int8_t* nst, int nkc,
                                         const DmaCtx& c, int t0, int k0, int8_t* dst, f32x16 (&acc)[4][2]) {
    const int lr = c.lane & 31;
#define TQ_MF(i, j) acc[i][j] = mfma_fp8(cur.w[i], cur.a[j], acc[i][j])
    TQ_MF(0, 0);
    nxt.w[0] = fp8_frag(nst, c.wn * 128 + 0 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0] + k0, dma_dst(c, dst, t0));
    TQ_SCHED_FENCE();
    TQ_MF(0, 1);
    nxt.w[1] = fp8_frag(nst, c.wn * 128 + 1 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 1] + k0, dma_dst(c, dst, t0 + 1));
    TQ_SCHED_FENCE();
    TQ_MF(1, 0);
    nxt.w[2] = fp8_frag(nst, c.wn * 128 + 2 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 2] + k0, dma_dst(c, dst, t0 + 2));
    TQ_SCHED_FENCE();
    TQ_MF(1, 1);
    nxt.w[3] = fp8_frag(nst, c.wn * 128 + 3 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 3] + k0, dma_dst(c, dst, t0 + 3));
    TQ_SCHED_FENCE();
    TQ_MF(2, 0);
    nxt.a[0] = fp8_frag(nst + kDmaW, c.wm * 64 + 0 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 4] + k0, dma_dst(c, dst, t0 + 4));
    TQ_SCHED_FENCE();
    TQ_MF(2, 1);
    nxt.a[1] = fp8_frag(nst + kDmaW, c.wm * 64 + 1 * 32 + lr, nkc, c.lane);
    dma16(c.src[t0 + 5] + k0, dma_dst(c, dst, t0 + 5));
    TQ_SCHED_FENCE();
    TQ_MF(3, 0);
    TQ_SCHED_FENCE();
    TQ_MF(3, 1);
    TQ_SCHED_FENCE();
#undef TQ_MF
}

__global__ __launch_bounds__(256, 1) void k_gemm_fp8_dma(const int8_t* __restrict__ qa,
                                                         const float* __restrict__ sa,
                                                         const int8_t* __restrict__ qw,
                                                         const float* __restrict__ sw,
                                                         const float* __restrict__ bias, int m, int n, int k,
                                                         float* __restrict__ y, int tiles_m, int tiles_n) {
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

    f32x16 acc[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = f32x16{};

    const int ks_n = k / kDmaBK;
    const int k_last = (ks_n - 1) * kDmaBK;  // stages past the end re-read the last one (never used)
#pragma unroll
    for (int t = 0; t < 12; ++t) dma16(c.src[t], dma_dst(c, lds, t));
#pragma unroll
    for (int t = 0; t < 12; ++t) dma16(c.src[t] + min(kDmaBK, k_last), dma_dst(c, lds + kDmaStage, t));
    asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
    Fp8Frags f0, f1;
    {
        const int lr = lane & 31;
#pragma unroll
        for (int i = 0; i < 4; ++i) f0.w[i] = fp8_frag(lds, c.wn * 128 + i * 32 + lr, 0, lane);
#pragma unroll
        for (int j = 0; j < 2; ++j) f0.a[j] = fp8_frag(lds + kDmaW, c.wm * 64 + j * 32 + lr, 0, lane);
    }
    // Ring: stage ks in buffer ks % 3; its 2 K chunks run as 2 steps.  The 12
    // DMAs of stage ks + 2 (into the buffer stage ks - 1 used) are split 6
    // before the barrier, 6 after.
    int rd = 0;
    for (int ks = 0; ks < ks_n; ++ks) {
        int8_t* st = lds + rd * kDmaStage;
        const int nrd = rd == 2 ? 0 : rd + 1;
        const int drd = nrd == 2 ? 0 : nrd + 1;
        int8_t* dst = lds + drd * kDmaStage;
        const int k0 = min((ks + 2) * kDmaBK, k_last);
        fp8_step(f0, f1, st, 1, c, 0, k0, dst, acc);
        // Stage ks + 1 has landed once at most the 6 DMAs just issued are
        // outstanding; after the barrier every wave is past its reads of buffer rd.
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
        fp8_step(f1, f0, lds + nrd * kDmaStage, 0, c, 6, k0, dst, acc);
        rd = nrd;
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    dma_epilogue(acc, c, lds, m0, n0, m, n, sa, sw, bias, nullptr, y);
}


// Skinny W8A8 for M <= 16 tokens (decode batches), K % 64 == 0: one block of 16
// waves per 16 weight rows, the waves splitting K into runs of kCPW 64-byte
// chunks.  Lane (q = l / 16, r16 = l % 16) loads 16 bytes at k = 64 c + 16 q of
// weight row r16 (the A operand of v_mfma_i32_16x16x64_i8) and of token r16's
// codes (the B operand, zero past M); A and B take a lane's bytes into the same
// k slots, so each MFMA adds the 64-k dot products of 16 rows x 16 tokens.  Every
// wave issues all of its loads at once.  A lane of the result holds D[4 q + e]
// [r16], e = 0..3: rows 4q..4q+3 for token r16.  The waves' int32 partials meet
// in LDS (exact, in any order) and the epilogue is the GEMM's, so acc and y equal
// the tiled kernels' bit for bit; 16 x 4096 tokens x weights in one round of
// 256 blocks instead of 16 blocks of 128 x 256 tiles.  K <= 8192 (kCPW <= 8).
constexpr int kSkinnyBlock = 1024, kSkinnyWaves = kSkinnyBlock / kWave;

template <int kCPW>
__global__ __launch_bounds__(kSkinnyBlock) void k_gemm_w8a8_skinny(const int8_t* __restrict__ qa,
                                                                   const float* __restrict__ sa,
                                                                   const int8_t* __restrict__ qw,
                                                                   const float* __restrict__ sw,
                                                                   const float* __restrict__ bias, int m, int n,
                                                                   int64_t k, int32_t* __restrict__ acc_out,
                                                                   float* __restrict__ y) {
    __shared__ i32x4 part[kSkinnyWaves][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int64_t C = k >> 6, c0 = static_cast<int64_t>(wave) * kCPW;
    const bool tok = r16 < m;
    const int8_t* wr = qw + (n0 + r16) * k + 16 * q;
    const int8_t* ar = qa + static_cast<int64_t>(tok ? r16 : 0) * k + 16 * q;
    i32x4 w[kCPW], a[kCPW];
#pragma unroll
    for (int i = 0; i < kCPW; ++i) {
        const int64_t c = min<int64_t>(c0 + i, C - 1);  // chunks past K: clamped, skipped below
        w[i] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wr + c * 64));
        a[i] = tok ? *reinterpret_cast<const i32x4*>(ar + c * 64) : i32x4{0, 0, 0, 0};
    }
    i32x4 d = i32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kCPW; ++i)
        if (c0 + i < C) d = mfma_i8(w[i], a[i], d);  // wave-uniform
    part[wave][lane] = d;
    __syncthreads();
    // thread t < 256: row t / 16, token t % 16 of the tile
    const int t = threadIdx.x;
    if (t < 256) {
        const int row = t >> 4, j = t & 15;
        const int e = row & 3, src = (row >> 2) * 16 + j;  // lane (q = row / 4, r16 = j), element row % 4
        int32_t v = 0;
#pragma unroll
        for (int wv = 0; wv < kSkinnyWaves; ++wv) v += part[wv][src][e];
        const int64_t nn = n0 + row;
        if (j < m) {
            if (acc_out) acc_out[static_cast<int64_t>(j) * n + nn] = v;
            y[static_cast<int64_t>(j) * n + nn] = fmaf(static_cast<float>(v) * sa[j], sw[nn], bias ? bias[nn] : 0.0f);
        }
    }
}


// The FP8 (e4m3) counterpart for M <= 16, K % 128 == 0: lanes take 32 bytes at k
// = 128 c + 32 q of their weight row and token (the A and B operands of the
// unscaled v_mfma_f32_16x16x128_f8f6f4; products exact in f32), f32 partials of
// the waves added in LDS in a fixed order, the GEMM's epilogue.  The sums run in
// another order than the tiled kernel's, so y agrees with it to f32 rounding.
// K <= 8192 (4 chunks per wave).
template <int kCPW>
__global__ __launch_bounds__(kSkinnyBlock) void k_gemm_fp8_skinny(const int8_t* __restrict__ qa,
                                                                  const float* __restrict__ sa,
                                                                  const int8_t* __restrict__ qw,
                                                                  const float* __restrict__ sw,
                                                                  const float* __restrict__ bias, int m, int n,
                                                                  int64_t k, float* __restrict__ y) {
    __shared__ f32x4 part[kSkinnyWaves][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int q = lane >> 4, r16 = lane & 15;
    const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 16;
    const int64_t C = k >> 7, c0 = static_cast<int64_t>(wave) * kCPW;
    const bool tok = r16 < m;
    const int8_t* wr = qw + (n0 + r16) * k + 32 * q;
    const int8_t* ar = qa + static_cast<int64_t>(tok ? r16 : 0) * k + 32 * q;
    i32x8 w[kCPW], a[kCPW];
#pragma unroll
    for (int i = 0; i < kCPW; ++i) {
        const int64_t c = min<int64_t>(c0 + i, C - 1);  // chunks past K: clamped, skipped below
        const i32x4 w0 = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wr + c * 128));
        const i32x4 w1 = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wr + c * 128 + 16));
        w[i] = i32x8{w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        i32x4 a0 = i32x4{0, 0, 0, 0}, a1 = a0;
        if (tok) {
            a0 = *reinterpret_cast<const i32x4*>(ar + c * 128);
            a1 = *reinterpret_cast<const i32x4*>(ar + c * 128 + 16);
        }
        a[i] = i32x8{a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
    }
    f32x4 d = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kCPW; ++i)
        if (c0 + i < C) d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(w[i], a[i], d, 0, 0, 0, 0, 0, 0);
    part[wave][lane] = d;
    __syncthreads();
    const int t = threadIdx.x;
    if (t < 256) {
        const int row = t >> 4, j = t & 15;
        const int e = row & 3, src = (row >> 2) * 16 + j;
        float v = 0.0f;
#pragma unroll
        for (int wv = 0; wv < kSkinnyWaves; ++wv) v += part[wv][src][e];
        const int64_t nn = n0 + row;
        if (j < m) y[static_cast<int64_t>(j) * n + nn] = fmaf(v * sa[j], sw[nn], bias ? bias[nn] : 0.0f);
    }
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" int tq_gemm_w8a8(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                            const float* bias, int64_t m, int64_t n, int64_t k, int32_t* acc,
                            float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemm_w8a8: negative shape");
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(sa && sw && y && (k == 0 || (qa && qw)), "tq_gemm_w8a8: null pointer");
    TQ_REQUIRE(aligned(sa, 4) && aligned(sw, 4) && aligned(y, 4) && (!acc || aligned(acc, 4)) &&
                   (!bias || aligned(bias, 4)),
               "tq_gemm_w8a8: misaligned pointer");
    // the MFMA kernels tile N by 16 rows, K by 16-byte vectors, and store 16-byte vectors
    if (k == 0 || n % 16 != 0 || k % 16 != 0 || !aligned(qa, 16) || !aligned(qw, 16) || !aligned(sw, 16) ||
        !aligned(y, 16) || (acc && !aligned(acc, 16)) || (bias && !aligned(bias, 16)))
        return launch_gemm_w8a8_generic(qa, sa, qw, sw, bias, m, n, k, acc, y, as_hip(stream));
    // decode batches: the skinny kernel, N / 16 blocks (K <= 8192: runs of up to 8
    // chunks per wave, whose loads all fit the registers)
    if (m <= 16 && k % 64 == 0 && k <= 8192 && n < (int64_t(1) << 31)) {
        const int64_t cpw = ((k >> 6) + kSkinnyWaves - 1) / kSkinnyWaves;
        const unsigned grid = static_cast<unsigned>(n / 16);
        const int mi = static_cast<int>(m), ni = static_cast<int>(n);
#define TQ_SKINNY(P) \
    k_gemm_w8a8_skinny<P><<<grid, kSkinnyBlock, 0, as_hip(stream)>>>(qa, sa, qw, sw, bias, mi, ni, k, acc, y)
        if (cpw <= 1)
            TQ_SKINNY(1);
        else if (cpw <= 2)
            TQ_SKINNY(2);
        else if (cpw <= 4)
            TQ_SKINNY(4);
        else
            TQ_SKINNY(8);
#undef TQ_SKINNY
        return check_launch("tq_gemm_w8a8");
    }
    if (k % kDmaBK == 0 && m < (int64_t(1) << 31) && n < (int64_t(1) << 31) && k < (int64_t(1) << 31)) {
        const int64_t tm = (m + kDmaBM - 1) / kDmaBM, tn = (n + kDmaBN - 1) / kDmaBN;
        if (tm * tn < (int64_t(1) << 31)) {
            k_gemm_w8a8_dma<false><<<static_cast<unsigned>(tm * tn), 256, 0, as_hip(stream)>>>(
                qa, sa, qw, sw, bias, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), acc, y,
                static_cast<int>(tm), static_cast<int>(tn));
            return check_launch("tq_gemm_w8a8");
        }
    }
    const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
    TQ_REQUIRE(tiles < (int64_t(1) << 31), "tq_gemm_w8a8: problem too large");
    k_gemm_w8a8<<<static_cast<unsigned>(tiles), kBlock, 0, as_hip(stream)>>>(qa, sa, qw, sw, bias, m, n, k, acc,
                                                                             y);
    return check_launch("tq_gemm_w8a8");
}

extern "C" int tq_gemm_fp8(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                           const float* bias, int64_t m, int64_t n, int64_t k, float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemm_fp8: negative shape");
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(sa && sw && y && (k == 0 || (qa && qw)), "tq_gemm_fp8: null pointer");
    TQ_REQUIRE(aligned(sa, 4) && aligned(sw, 4) && aligned(y, 4) && (!bias || aligned(bias, 4)),
               "tq_gemm_fp8: misaligned pointer");
    // the MFMA kernel takes K in 128-byte stages, stores 4 consecutive n per lane
    // (N % 16 == 0) and loads 16-byte vectors
    const bool fast = k > 0 && k % kDmaBK == 0 && n % 16 == 0 && aligned(qa, 16) && aligned(qw, 16) &&
                      aligned(sw, 16) && aligned(y, 16) && (!bias || aligned(bias, 16)) &&
                      m < (int64_t(1) << 31) && n < (int64_t(1) << 31) && k < (int64_t(1) << 31);
    if (fast && m <= 16 && k <= 8192) {  // decode batches: the skinny kernel, N / 16 blocks
        const int64_t cpw = ((k >> 7) + kSkinnyWaves - 1) / kSkinnyWaves;
        const unsigned grid = static_cast<unsigned>(n / 16);
        const auto* a = reinterpret_cast<const int8_t*>(qa);
        const auto* w = reinterpret_cast<const int8_t*>(qw);
        const int mi = static_cast<int>(m), ni = static_cast<int>(n);
        if (cpw <= 1)
            k_gemm_fp8_skinny<1><<<grid, kSkinnyBlock, 0, as_hip(stream)>>>(a, sa, w, sw, bias, mi, ni, k, y);
        else if (cpw <= 2)
            k_gemm_fp8_skinny<2><<<grid, kSkinnyBlock, 0, as_hip(stream)>>>(a, sa, w, sw, bias, mi, ni, k, y);
        else
            k_gemm_fp8_skinny<4><<<grid, kSkinnyBlock, 0, as_hip(stream)>>>(a, sa, w, sw, bias, mi, ni, k, y);
        return check_launch("tq_gemm_fp8");
    }
    if (fast) {
        const int64_t tm = (m + kDmaBM - 1) / kDmaBM, tn = (n + kDmaBN - 1) / kDmaBN;
        if (tm * tn < (int64_t(1) << 31)) {
            k_gemm_fp8_dma<<<static_cast<unsigned>(tm * tn), 256, 0, as_hip(stream)>>>(
                reinterpret_cast<const int8_t*>(qa), sa, reinterpret_cast<const int8_t*>(qw), sw, bias,
                static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), y, static_cast<int>(tm),
                static_cast<int>(tn));
            return check_launch("tq_gemm_fp8");
        }
    }
    return launch_gemm_fp8_generic(qa, sa, qw, sw, bias, m, n, k, y, as_hip(stream));
}
