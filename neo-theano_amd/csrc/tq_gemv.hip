// tq_gemv.hip -- decode-shaped 8-bit weight-only quantized Linear
// (y = x . dequant(W)^T + b) for gfx950, the reference's Linear::forward
// (crates/theano-nn/src/linear.rs:111-121) over the dequantized weight of
// quantize.rs:22-27.  One kernel body serves per-row INT8 codes and per-row
// FP8 (OCP e4m3) codes; only the byte -> f32 decode differs.
//
// HBM-bound weight stream.  The grid is persistent: every
// wave owns a contiguous range of output rows, keeps its slice of x in
// registers for its whole life (staged once per block through LDS), and keeps
// the loads of the next kRows rows in flight (global_load_dwordx4,
// non-temporal).  Lane l owns 16-byte slices of a row at byte 16*l of every
// 1 KB chunk, so each wave-wide load is 1 KB contiguous; a row's partial dot
// products meet in one wave64 butterfly.  Up to 4 tokens per pass.
#include "tq_internal.h"
#include "tq_rowfmt.h"

namespace tq {
namespace {

__device__ __forceinline__ int64_t uniform(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(v));
    const uint32_t hi = __builtin_amdgcn_readfirstlane(static_cast<uint32_t>(static_cast<uint64_t>(v) >> 32));
    return static_cast<int64_t>((static_cast<uint64_t>(hi) << 32) | lo);
}


// Byte codes -> f32 values: 4 codes of a little-endian word.
struct CodeI8 {
    typedef int8_t code_t;
    __device__ static void decode4(int w, float (&v)[4]) {
#pragma unroll
        for (int b = 0; b < 4; ++b) v[b] = static_cast<float>(static_cast<int8_t>((w >> (8 * b)) & 0xFF));
    }
};

struct CodeFp8 {
    typedef uint8_t code_t;
    __device__ static void decode4(int w, float (&v)[4]) {
        v[0] = __builtin_amdgcn_cvt_f32_fp8(w, 0);
        v[1] = __builtin_amdgcn_cvt_f32_fp8(w, 1);
        v[2] = __builtin_amdgcn_cvt_f32_fp8(w, 2);
        v[3] = __builtin_amdgcn_cvt_f32_fp8(w, 3);
    }
};

// ------------------------------------------------------------------ kernel
// Chunk c covers k in [1024c, 1024c + 1024): lane l owns the 16 codes at
// k = 1024c + 16l.  y = s[row] * sum(value(q) * x) + b.
//
// kWB waves per block, 8 / kWB blocks per CU (persistent): 4-wave blocks, two
// per CU, at one token (each block stages x itself; 4.6 against 4.75 us at
// 4096 x 4096), one 8-wave block per CU beyond (x of several tokens staged
// twice per CU costs more than it gains).  With kKS = 1 every wave
// owns a contiguous run of rows and all of K; with kKS = 2 the waves pair up:
// both waves of a pair own the same run of rows, the first takes chunks
// 0 .. kC0 - 1 and the second the rest, so each holds half of x in registers
// (that is what lets 3-4 tokens at K = 4096, or 2 at K = 8192, run in one
// pass).  A wave first issues the weight loads of its first kRows rows
// (unconditional: rows past its run re-read its last row and are not
// stored), then the block stages x in LDS once (f32, K-contiguous per token)
// and every lane copies its 16-value slices into registers; rows are then
// consumed kRows at a time.  The next group's loads go out once the current
// group's have landed, before its arithmetic: one group in flight per wave.
// With every wave's next rows requested at once (8 KB per wave, the whole
// 16.8 MB weight of a 4096 x 4096 layer in flight) the same GEMV took 5.13
// against 4.63 us.  x crosses L2 once per block instead of once per
// wave.  A pair's two partial sums of a row meet in LDS after the row loop
// and are added in a fixed order (first half + second half).
// LDS slot of x item j (4 values) of a token: item 4l + e of a 256-item chunk is
// lane l's e-th 16-byte slice, and e is xor-ed with bits 2-3 of l, so that the
// 64 lanes' reads of one e fall in distinct banks (lanes 64 bytes apart collide
// 16-way unswizzled).
__device__ __forceinline__ int xslot(int j) { return j ^ ((j >> 4) & 3); }
constexpr int kMaxPairRows = 64;  // rows per wave pair that the LDS partial sums hold

template <class Code, int kM, int kChunks, int kRows, int kKS, int kWB>
__global__ __launch_bounds__(64 * kWB, 8 / kWB) void k_gemv_w8(const float* __restrict__ x, int64_t x_stride,
                                                      const typename Code::code_t* __restrict__ q,
                                                      const float* __restrict__ s,
                                                      const float* __restrict__ bias, int64_t n,
                                                      int64_t k, float* __restrict__ y,
                                                      int64_t y_stride, int64_t rows_per_wave) {
    static_assert(kKS == 1 || kKS == 2, "K split over one or two waves");
    constexpr int kBlk = 64 * kWB;
    constexpr int kC0 = (kChunks + kKS - 1) / kKS;  // chunks of the first (or only) wave of a pair
    __shared__ f32x4 xs[kM][kChunks * 256];
    __shared__ float part[kKS == 2 ? kWB : 1][kKS == 2 ? kMaxPairRows : 1][kM];
    const int lane = threadIdx.x & (kWave - 1);
    const int wv = threadIdx.x >> 6;
    const int half = kKS == 2 ? (wv & 1) : 0;
    // chunks [cb, cb + nc) of every row; the second wave of a pair may have fewer
    const int cb = half * kC0, nc = half == 0 ? kC0 : kChunks - kC0;
    const int64_t wave = uniform(static_cast<int64_t>(blockIdx.x) * (kWB / kKS) + wv / kKS);
    const int64_t row_begin = wave * rows_per_wave;
    const int64_t row_end = min(n, row_begin + rows_per_wave);
    const int64_t row_last = max(row_begin, row_end - 1);  // clamp target (valid when the run is empty too)
    const int64_t row_clamp = min(row_last, n - 1);

    auto load_rows = [&](int64_t row0, i32x4 (&wq)[kRows][kC0]) {
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int c = 0; c < kC0; ++c) {
                const int64_t row = min(row0 + r, row_clamp);
                const int64_t kb = min<int64_t>(1024 * (cb + min(c, nc - 1)) + 16 * lane, k - 16);
                wq[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(q + row * k + kb));
            }
    };
    // x first (vmcnt completes in order: staging x then waits for x alone, not for
    // the weight rows issued after it), then the first rows, then x -> LDS (zero
    // past K) and each lane's 16-value slices -> registers
    const int k4 = static_cast<int>(k >> 2);
    constexpr int kXItems = kM * kChunks * 256, kXPer = (kXItems + kBlk - 1) / kBlk;
    f32x4 xv[kXPer];
#pragma unroll
    for (int qi = 0; qi < kXPer; ++qi) {
        const int i = threadIdx.x + qi * kBlk;
        const int m = i / (kChunks * 256), j = i - m * (kChunks * 256);
        xv[qi] = i < kXItems && j < k4 ? *reinterpret_cast<const f32x4*>(x + m * x_stride + 4 * j)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    i32x4 wa[kRows][kC0], wb[kRows][kC0];
    load_rows(row_begin, wa);
#pragma unroll
    for (int qi = 0; qi < kXPer; ++qi) {
        const int i = threadIdx.x + qi * kBlk;
        const int m = i / (kChunks * 256), j = i - m * (kChunks * 256);
        if (i < kXItems) xs[m][xslot(j)] = xv[qi];
    }
    __syncthreads();
    float xr[kM][kC0][16];
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int c = 0; c < kC0; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // the second wave's chunks past nc read zeros' stand-in (never used)
                const f32x4 v = xs[m][xslot(min(cb + c, kChunks - 1) * 256 + 4 * lane + j)];
                xr[m][c][4 * j + 0] = v.x;
                xr[m][c][4 * j + 1] = v.y;
                xr[m][c][4 * j + 2] = v.z;
                xr[m][c][4 * j + 3] = v.w;
            }

    // the kRows rows at row0 from the registers `cur` (stores past the run skipped)
    auto group = [&](int64_t row0, const i32x4 (&cur)[kRows][kC0]) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            float acc[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[m] = 0.0f;
#pragma unroll
            for (int c = 0; c < kC0; ++c) {
                if (c >= nc) break;  // uniform: the second wave of a pair with fewer chunks
                const int words[4] = {cur[r][c].x, cur[r][c].y, cur[r][c].z, cur[r][c].w};
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float wv4[4];
                    Code::decode4(words[j], wv4);
#pragma unroll
                    for (int b = 0; b < 4; ++b)
#pragma unroll
                        for (int m = 0; m < kM; ++m) acc[m] = fmaf(wv4[b], xr[m][c][4 * j + b], acc[m]);
                }
            }
            const int64_t row = row0 + r;
            if constexpr (kKS == 1) {
                // scale and bias read at a wave-uniform address (scalar loads): a bias
                // read under the lane-0 store condition became a vector load whose
                // wait, hoisted ahead of the arithmetic, also waited for every
                // weight load in flight
                const int64_t rc = min(row, row_clamp);
                const float sc = s[rc];
                const float bb = bias ? bias[rc] : 0.0f;
#pragma unroll
                for (int m = 0; m < kM; ++m) {
                    const float v = wave_sum(acc[m]);
                    if (lane == 0 && row < row_end) y[m * y_stride + row] = sc * v + bb;
                }
            } else {
#pragma unroll
                for (int m = 0; m < kM; ++m) {
                    const float v = wave_sum(acc[m]);
                    if (lane == 0 && row < row_end) part[wv][row - row_begin][m] = v;
                }
            }
        }
    };
    // Row groups alternate between two register buffers, the next group's loads
    // issued before the current group's arithmetic.  The arithmetic reads the
    // buffers in place: a copy of a register whose load is in flight waits for
    // that load, which would make every group wait for all of its loads.
    for (int64_t row0 = row_begin;;) {
        if (row0 + kRows >= row_end) {
            group(row0, wa);
            break;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the current group has landed
        load_rows(row0 + kRows, wb);
        group(row0, wa);
        row0 += kRows;
        if (row0 + kRows >= row_end) {
            group(row0, wb);
            break;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        load_rows(row0 + kRows, wa);
        group(row0, wb);
        row0 += kRows;
    }
    if constexpr (kKS == 2) {
        __syncthreads();
        // the first wave of each pair adds the two halves of its rows
        if (half == 0) {
            for (int i = lane; i < (row_end - row_begin) * kM; i += kWave) {
                const int ri = i / kM, m = i - ri * kM;
                const int64_t row = row_begin + ri;
                const float v = part[wv][ri][m] + part[wv + 1][ri][m];
                y[m * y_stride + row] = s[row] * v + (bias ? bias[row] : 0.0f);
            }
        }
    }
}

// ------------------------------------------- W8A8 / FP8 with fused activations
// The decode form of quantize(x) + W8A8 GEMM in one kernel: every block stages
// the (few) activation rows in LDS, computes their per-row absmax and scale and
// codes them exactly as tq_quantize_{i8,fp8}_rowwise do, then streams weight
// rows as k_gemv_w8.  INT8: v_dot4 int32 dot products of the codes (exact, the
// GEMM's accumulators); FP8: f32 FMAs of the e4m3 values.  Epilogue as the
// GEMM's: y = (f32(acc) * s_a) * s_w (+ b).
template <class Fmt>
struct A8;
template <>
struct A8<FmtI8> {
    typedef int32_t acc_t;
    typedef uint32_t xreg_t;  // 4 codes
    __device__ static void encode(const FmtI8::Row& r, f32x4 v, xreg_t* out) { out[0] = r.code4(v); }
    __device__ static f32x4 pack(const xreg_t* e) { return f32x4{__uint_as_float(e[0]), 0.f, 0.f, 0.f}; }
    __device__ static void unpack(const f32x4& v, xreg_t* e) { e[0] = __float_as_uint(v.x); }
    static constexpr int kRegsPer4 = 1;
    __device__ static void dot16(const i32x4& w, const xreg_t* x, acc_t& acc) {
        acc = __builtin_amdgcn_sdot4(w.x, static_cast<int>(x[0]), acc, false);
        acc = __builtin_amdgcn_sdot4(w.y, static_cast<int>(x[1]), acc, false);
        acc = __builtin_amdgcn_sdot4(w.z, static_cast<int>(x[2]), acc, false);
        acc = __builtin_amdgcn_sdot4(w.w, static_cast<int>(x[3]), acc, false);
    }
    __device__ static float total(acc_t a) { return static_cast<float>(wave_sum(a)); }
};
template <>
struct A8<FmtFp8> {
    typedef float acc_t;
    typedef float xreg_t;  // e4m3 values (the codes without the row scale)
    __device__ static void encode(const FmtFp8::Row& r, f32x4 v, xreg_t* out) {
        const f32x4 e = FmtFp8::value4(r.code4(v), 1.0f);
        out[0] = e.x;
        out[1] = e.y;
        out[2] = e.z;
        out[3] = e.w;
    }
    __device__ static f32x4 pack(const xreg_t* e) { return f32x4{e[0], e[1], e[2], e[3]}; }
    __device__ static void unpack(const f32x4& v, xreg_t* e) {
        e[0] = v.x;
        e[1] = v.y;
        e[2] = v.z;
        e[3] = v.w;
    }
    static constexpr int kRegsPer4 = 4;
    __device__ static void dot16(const i32x4& w, const xreg_t* x, acc_t& acc) {
        const int words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float wv[4];
            CodeFp8::decode4(words[j], wv);
#pragma unroll
            for (int b = 0; b < 4; ++b) acc = fmaf(wv[b], x[4 * j + b], acc);
        }
    }
    __device__ static float total(acc_t a) { return wave_sum(a); }
};

template <class Fmt, int kM, int kChunks, int kRows, int kWB>
__global__ __launch_bounds__(64 * kWB, 8 / kWB) void k_gemv_a8(const float* __restrict__ x, int64_t x_stride,
                                                      const typename Fmt::code_t* __restrict__ q,
                                                      const float* __restrict__ s, const float* __restrict__ bias,
                                                      int64_t n, int64_t k, float* __restrict__ y, int64_t y_stride,
                                                      int64_t rows_per_wave) {
    using P = A8<Fmt>;
    constexpr int kBlk = 64 * kWB;
    __shared__ f32x4 xs[kM][kChunks * 256];
    __shared__ float red[kWB][kM];
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x >> 6;
    const int64_t wave = uniform(static_cast<int64_t>(blockIdx.x) * kWB + wv);
    const int64_t row_begin = wave * rows_per_wave;
    const int64_t row_end = min(n, row_begin + rows_per_wave);
    const int64_t row_last = max(row_begin, row_end - 1);
    const int64_t row_clamp = min(row_last, n - 1);

    auto load_rows = [&](int64_t row0, i32x4 (&wq)[kRows][kChunks]) {
#pragma unroll
        for (int r = 0; r < kRows; ++r)
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                const int64_t row = min(row0 + r, row_clamp);
                const int64_t kb = min<int64_t>(1024 * c + 16 * lane, k - 16);
                wq[r][c] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(q + row * k + kb));
            }
    };
    // x first (vmcnt completes in order: the absmax and coding of x then wait for x
    // alone, not for the weight rows issued after it), then the first rows
    const int k4 = static_cast<int>(k >> 2);
    constexpr int kXItems = kM * kChunks * 256, kXPer = (kXItems + kBlk - 1) / kBlk;
    f32x4 xv[kXPer];
#pragma unroll
    for (int qi = 0; qi < kXPer; ++qi) {
        const int i = threadIdx.x + qi * kBlk;
        const int m = i / (kChunks * 256), j = i - m * (kChunks * 256);
        xv[qi] = i < kXItems && j < k4 ? *reinterpret_cast<const f32x4*>(x + m * x_stride + 4 * j)
                                       : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    i32x4 wa[kRows][kChunks], wb[kRows][kChunks];
    load_rows(row_begin, wa);

    // x -> LDS (zero past K) and the NaN-ignoring absmax of each row over its K values
    float mx[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) mx[m] = -INFINITY;
#pragma unroll
    for (int qi = 0; qi < kXPer; ++qi) {
        const int i = threadIdx.x + qi * kBlk;
        if (i >= kXItems) continue;
        const int m = i / (kChunks * 256), j = i - m * (kChunks * 256);
        const f32x4 v = xv[qi];
        xs[m][xslot(j)] = v;
        if (j < k4) {
            const float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
#pragma unroll
            for (int mm = 0; mm < kM; ++mm)
                if (mm == m) mx[mm] = fmaxf(mx[mm], a);
        }
    }
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        const float w = wave_max(mx[m]);
        if (lane == 0) red[wv][m] = w;
    }
    __syncthreads();
    float sa[kM];
#pragma unroll
    for (int m = 0; m < kM; ++m) {
        float r = red[0][m];
#pragma unroll
        for (int i = 1; i < kWB; ++i) r = fmaxf(r, red[i][m]);
        sa[m] = row_scale<Fmt>(absmax_finish(r));
    }
    // the block codes each 4-value entry once (in place in LDS, slot by slot), then
    // every lane copies its 16-value slices into registers
    for (int i = threadIdx.x; i < kM * kChunks * 256; i += kBlk) {
        const int m = i / (kChunks * 256), j = i - m * (kChunks * 256);
        typename P::xreg_t e[P::kRegsPer4];
        float sm = sa[0];
#pragma unroll
        for (int mm = 1; mm < kM; ++mm) sm = mm == m ? sa[mm] : sm;
        P::encode(typename Fmt::Row(sm), xs[m][j], e);
        xs[m][j] = P::pack(e);
    }
    __syncthreads();
    typename P::xreg_t xr[kM][kChunks][4 * P::kRegsPer4];
#pragma unroll
    for (int m = 0; m < kM; ++m)
#pragma unroll
        for (int c = 0; c < kChunks; ++c)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                P::unpack(xs[m][xslot(c * 256 + 4 * lane + j)], &xr[m][c][j * P::kRegsPer4]);
    if (row_begin >= row_end) return;

    auto group = [&](int64_t row0, const i32x4 (&cur)[kRows][kChunks]) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            typename P::acc_t acc[kM];
#pragma unroll
            for (int m = 0; m < kM; ++m) acc[m] = 0;
#pragma unroll
            for (int c = 0; c < kChunks; ++c)
#pragma unroll
                for (int m = 0; m < kM; ++m) P::dot16(cur[r][c], xr[m][c], acc[m]);
            const int64_t row = row0 + r;
            const int64_t rc = min(row, row_clamp);
            const float sc = s[rc];
            const float bb = bias ? bias[rc] : 0.0f;  // wave-uniform, as in k_gemv_w8
#pragma unroll
            for (int m = 0; m < kM; ++m) {
                const float v = P::total(acc[m]);
                if (lane == 0 && row < row_end) y[m * y_stride + row] = fmaf(v * sa[m], sc, bb);
            }
        }
    };
    // two register buffers in turn, read in place, the next group requested once
    // the current one has landed (as in k_gemv_w8)
    for (int64_t row0 = row_begin;;) {
        if (row0 + kRows >= row_end) {
            group(row0, wa);
            break;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        load_rows(row0 + kRows, wb);
        group(row0, wa);
        row0 += kRows;
        if (row0 + kRows >= row_end) {
            group(row0, wb);
            break;
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        load_rows(row0 + kRows, wa);
        group(row0, wb);
        row0 += kRows;
    }
}

// Persistent grid: blocks_per_cu blocks per CU (fewer if there are few rows),
// contiguous row runs per wave (or wave pair: `runs_per_block` runs per block),
// a multiple of kRows each.
template <int kRows>
void grid_for_rows(int64_t n, int64_t* blocks, int64_t* rows_per_wave, int runs_per_block, int64_t max_rows,
                   int blocks_per_cu) {
    const int64_t slots = static_cast<int64_t>(device_cu_count()) * blocks_per_cu * runs_per_block;
    int64_t waves = (n + kRows - 1) / kRows;
    if (waves > slots) waves = slots;
    if ((n + waves - 1) / waves > max_rows) waves = (n + max_rows - 1) / max_rows;  // more blocks than CUs
    int64_t rpw = (n + waves - 1) / waves;
    rpw = (rpw + kRows - 1) / kRows * kRows;
    *rows_per_wave = rpw;
    waves = (n + rpw - 1) / rpw;
    *blocks = (waves + runs_per_block - 1) / runs_per_block;
}

// Rows per group: two, unless the x slices held in registers (16 values per
// token and chunk) would leave no room for two double-buffered groups of
// weight rows (the compiler then spills): one at kM * kChunks > 4.
constexpr int rows_in_flight(int x_regs) { return x_regs <= 64 ? 2 : 1; }

// Token counts and K chunks a pass runs together (the dispatch below never asks
// for more).  Weight-only GEMV (x split over a wave pair beyond one token): 4
// tokens up to K = 4096, 2 up to 8192.  Fused-activation GEMV (no split): 4
// tokens up to K = 2048, 2 up to 4096, 1 beyond.
constexpr bool pass_shape_w8(int m, int chunks) { return m <= 4 && (chunks <= 4 || m <= 2); }
constexpr bool pass_shape(int m, int chunks) { return m * chunks <= 8 && (m <= 2 || chunks <= 2); }

// K split over a wave pair once x would take more than 128 registers per lane
// (3-4 tokens at K = 4096, 2 at K = 8192): one pass instead of two.  Measured
// at 2 tokens and K = 4096, where the split is not needed, it is slower (6.7
// against 6.0 us), so smaller shapes keep every wave on all of K.
constexpr int ks_for(int m, int chunks) { return (m >= 2 && m * chunks > 8) ? 2 : 1; }

template <class Code, int kM, int kChunks>
void launch_w8(const float* x, int64_t xs, const typename Code::code_t* q, const float* s, const float* b,
               int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    constexpr int kKS = ks_for(kM, kChunks);
    // one token: groups of one row (the next row requested once the current one
    // has landed) in 4-wave blocks, two per CU
    constexpr int kRows = kM == 1 ? 1 : rows_in_flight(kM * ((kChunks + kKS - 1) / kKS) * 16);
    constexpr int kWB = kM == 1 ? 4 : 8;
    int64_t blocks, rpw;
    static_assert(kMaxPairRows % kRows == 0, "row runs are whole row groups");
    grid_for_rows<kRows>(n, &blocks, &rpw, kWB / kKS, kKS == 2 ? kMaxPairRows : INT64_MAX, 8 / kWB);
    k_gemv_w8<Code, kM, kChunks, kRows, kKS, kWB><<<static_cast<unsigned>(blocks), 64 * kWB, 0, st>>>(
        x, xs, q, s, b, n, k, y, ys, rpw);
}

template <class Code, int kM, int kChunks = 1>
void dispatch_w8(int chunks, const float* x, int64_t xs, const typename Code::code_t* q, const float* s,
                 const float* b, int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    if constexpr (kChunks < 8 && pass_shape_w8(kM, kChunks + 1)) {
        if (chunks > kChunks) return dispatch_w8<Code, kM, kChunks + 1>(chunks, x, xs, q, s, b, n, k, y, ys, st);
    }
    launch_w8<Code, kM, kChunks>(x, xs, q, s, b, n, k, y, ys, st);
}

template <class Fmt, int kM, int kChunks>
void launch_a8(const float* x, int64_t xs, const typename Fmt::code_t* q, const float* s, const float* b, int64_t n,
               int64_t k, float* y, int64_t ys, hipStream_t st) {
    // one token: one row per group in 4-wave blocks, two per CU (as the weight-only GEMV)
    constexpr int kRows = kM == 1 ? 1 : rows_in_flight(kM * kChunks * 4 * A8<Fmt>::kRegsPer4);
    constexpr int kWB = kM == 1 ? 4 : 8;
    int64_t blocks, rpw;
    grid_for_rows<kRows>(n, &blocks, &rpw, kWB, INT64_MAX, 8 / kWB);
    k_gemv_a8<Fmt, kM, kChunks, kRows, kWB><<<static_cast<unsigned>(blocks), 64 * kWB, 0, st>>>(x, xs, q, s, b, n, k,
                                                                                              y, ys, rpw);
}

template <class Fmt, int kM, int kChunks = 1>
void dispatch_a8(int chunks, const float* x, int64_t xs, const typename Fmt::code_t* q, const float* s,
                 const float* b, int64_t n, int64_t k, float* y, int64_t ys, hipStream_t st) {
    if constexpr (kChunks < 8 && pass_shape(kM, kChunks + 1)) {
        if (chunks > kChunks) return dispatch_a8<Fmt, kM, kChunks + 1>(chunks, x, xs, q, s, b, n, k, y, ys, st);
    }
    launch_a8<Fmt, kM, kChunks>(x, xs, q, s, b, n, k, y, ys, st);
}

// Activations quantized in place: K % 16 == 0, K <= 8192, x and q 16-byte
// aligned.  Other shapes are rejected (TQ_EINVAL); callers run
// tq_quantize_*_rowwise + tq_gemm_* for them.
template <class Fmt>
int gemv_a8(const float* x, int64_t m, const typename Fmt::code_t* q, const float* s, const float* bias, int64_t n,
            int64_t k, float* y, hipStream_t st, const char* what) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "%s: negative shape", what);
    TQ_REQUIRE(m <= 16, "%s: M=%lld > 16 (decode shapes)", what, (long long)m);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(x && q && s && y, "%s: null pointer", what);
    TQ_REQUIRE(k > 0 && k % 16 == 0 && k <= 8 * 1024, "%s: K=%lld must be a positive multiple of 16 up to 8192", what,
               (long long)k);
    TQ_REQUIRE(aligned(x, 16) && aligned(q, 16) && aligned(s, 4) && aligned(y, 4) && (!bias || aligned(bias, 4)),
               "%s: x and q must be 16-byte aligned, f32 pointers 4-byte aligned", what);
    const int chunks = static_cast<int>((k + 1023) / 1024);
    const int64_t per_pass = chunks <= 2 ? 4 : (chunks <= 4 ? 2 : 1);
    for (int64_t m0 = 0; m0 < m; m0 += per_pass) {
        const int64_t mm = (m - m0) < per_pass ? (m - m0) : per_pass;
        const float* xp = x + m0 * k;
        float* yp = y + m0 * n;
        if (mm == 1) dispatch_a8<Fmt, 1>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 2) dispatch_a8<Fmt, 2>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 3) dispatch_a8<Fmt, 3>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else dispatch_a8<Fmt, 4>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        const int rc = check_launch(what);
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

template <class Code>
int gemv_8bit(const float* x, int64_t m, const typename Code::code_t* q, const float* s, const float* bias,
              int64_t n, int64_t k, float* y, hipStream_t st, const char* what) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "%s: negative shape", what);
    TQ_REQUIRE(m <= 16, "%s: M=%lld > 16 (decode shapes; run longer inputs in chunks)", what, (long long)m);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(y, "%s: null y", what);
    TQ_REQUIRE(k == 0 || (x && q), "%s: null pointer", what);
    TQ_REQUIRE(s, "%s: null scales", what);
    TQ_REQUIRE(aligned(x, 4) && aligned(s, 4) && (!bias || aligned(bias, 4)) && aligned(y, 4),
               "%s: misaligned f32 pointer", what);
    // the tuned kernel streams 16-byte vectors of K-contiguous rows held in registers
    if (k == 0 || k % 16 != 0 || k > 8 * 1024 || !aligned(x, 16) || !aligned(q, 16))
        return launch_linear_8bit_generic(x, m, q, s, bias, n, k, y, st);
    const int chunks = static_cast<int>((k + 1023) / 1024);
    const int64_t per_pass = chunks <= 4 ? 4 : 2;
    for (int64_t m0 = 0; m0 < m; m0 += per_pass) {
        const int64_t mm = (m - m0) < per_pass ? (m - m0) : per_pass;
        const float* xp = x + m0 * k;
        float* yp = y + m0 * n;
        if (mm == 1) dispatch_w8<Code, 1>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 2) dispatch_w8<Code, 2>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else if (mm == 3) dispatch_w8<Code, 3>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        else dispatch_w8<Code, 4>(chunks, xp, k, q, s, bias, n, k, yp, n, st);
        const int rc = check_launch(what);
        if (rc != TQ_OK) return rc;
    }
    return TQ_OK;
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_gemv_w8(const float* x, int64_t m, const int8_t* q, const float* s, const float* bias,
               int64_t n, int64_t k, float* y, tq_stream_t stream) {
    return gemv_8bit<CodeI8>(x, m, q, s, bias, n, k, y, as_hip(stream), "tq_gemv_w8");
}

int tq_gemv_fp8(const float* x, int64_t m, const uint8_t* q, const float* s, const float* bias,
                int64_t n, int64_t k, float* y, tq_stream_t stream) {
    return gemv_8bit<CodeFp8>(x, m, q, s, bias, n, k, y, as_hip(stream), "tq_gemv_fp8");
}

int tq_gemv_w8a8(const float* x, int64_t m, const int8_t* qw, const float* sw, const float* bias, int64_t n,
                 int64_t k, float* y, tq_stream_t stream) {
    return gemv_a8<FmtI8>(x, m, qw, sw, bias, n, k, y, as_hip(stream), "tq_gemv_w8a8");
}

int tq_gemv_fp8a8(const float* x, int64_t m, const uint8_t* qw, const float* sw, const float* bias, int64_t n,
                  int64_t k, float* y, tq_stream_t stream) {
    return gemv_a8<FmtFp8>(x, m, qw, sw, bias, n, k, y, as_hip(stream), "tq_gemv_fp8a8");
}

}  // extern "C"
