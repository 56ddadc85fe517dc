// tq_gemm.hip -- prefill-shaped W8A8 quantized Linear on gfx950 i8 MFMA.
//
//   acc[m, n] = sum_k qa[m, k] * qw[n, k]          (int32, exact)
//   y[m, n]   = f32(acc) * sa[m] * sw[n] (+ b[n])
//
// The reference value is Tensor::mm over the dequantized operands
// (crates/theano-core/src/tensor_ops.rs:379-410); over integral f64 codes that
// product is exact, so acc is bit-exact with it.
//
// Both operands are K-contiguous ("NT"), which is the layout v_mfma_i32_16x16x64_i8
// wants for A and B alike.  A block owns a 128 (n) x 128 (m) output tile and
// walks K in 128-byte slices staged through LDS (rows padded to 144 B against
// bank conflicts); the next slice is prefetched into registers while the
// current one feeds the matrix cores.  Weights are the MFMA A operand so that
// each lane's four accumulator rows are four consecutive n: the epilogue
// stores 16-byte vectors of y and acc.
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
            o.x = static_cast<float>(c.x) * s_row * swv.x + bv.x;
            o.y = static_cast<float>(c.y) * s_row * swv.y + bv.y;
            o.z = static_cast<float>(c.z) * s_row * swv.z + bv.z;
            o.w = static_cast<float>(c.w) * s_row * swv.w + bv.w;
            *reinterpret_cast<f32x4*>(y + mm * n + nb) = o;
        }
    }
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" int tq_gemm_w8a8(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                            const float* bias, int64_t m, int64_t n, int64_t k, int32_t* acc,
                            float* y, tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemm_w8a8: negative shape");
    TQ_REQUIRE(n % 16 == 0, "tq_gemm_w8a8: N=%lld is not a multiple of 16", (long long)n);
    TQ_REQUIRE(k % 16 == 0, "tq_gemm_w8a8: K=%lld is not a multiple of 16", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(k > 0, "tq_gemm_w8a8: K=0");
    TQ_REQUIRE(qa && sa && qw && sw && y, "tq_gemm_w8a8: null pointer");
    TQ_REQUIRE(aligned(qa, 16) && aligned(qw, 16) && aligned(sw, 16) && aligned(y, 16) &&
                   (!acc || aligned(acc, 16)) && (!bias || aligned(bias, 16)) && aligned(sa, 4),
               "tq_gemm_w8a8: misaligned pointer (qa, qw, sw, bias, y, acc need 16 B)");
    const int64_t tiles = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
    TQ_REQUIRE(tiles < (int64_t(1) << 31), "tq_gemm_w8a8: problem too large");
    k_gemm_w8a8<<<static_cast<unsigned>(tiles), kBlock, 0, as_hip(stream)>>>(qa, sa, qw, sw, bias, m, n, k, acc,
                                                                             y);
    return check_launch("tq_gemm_w8a8");
}
