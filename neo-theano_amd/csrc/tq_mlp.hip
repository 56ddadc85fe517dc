// tq_mlp.hip -- prefill-shaped INT4 group-128 Linear (W4A16) and the quantized
// Llama-style FFN on gfx950 bf16 MFMA.
//
// Reference composition: Linear::forward (crates/theano-nn/src/linear.rs:111-121)
// over dequantized weights, SiLU (crates/theano-nn/src/activation.rs:66-79,
// x * 1/(1+exp(-x))) and Tensor::mul, all in f64; here f32 accumulation.
//
// Weight nibbles go to bf16 in registers: after xor 0x8 a nibble holds q+8, and
// (q+8) | 0x4300 is the bf16 of 136+q.  The MFMA therefore accumulates
// sum (136+q)*x over each 128-long group; the kernel subtracts 136*sum(x) of
// the group (exact operands, f32 sums) and applies the f16 group scale once
// per group: y += s_g * (T_g - 136 X_g).  The pairing of nibbles inside a
// dword, (k, k+4), (k+1, k+5), ..., is matched by storing activations in LDS
// in the same order within every 8-element block.
//
// The down projection takes the f32 intermediate h = SiLU(g)*u; it is split
// into bf16 hi + lo (h - hi is exact in f32, its bf16 rounding leaves ~2^-17
// relative error) and both halves go through the MFMA.
#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kBlock = 256;
constexpr int kTileN = 128;           // weight rows per block (gate+up: 64 + 64)
constexpr int kWRow = 64 + 16;        // LDS bytes per packed weight row (+pad)
constexpr int kARow = 256 + 16;       // LDS bytes per activation row of 128 bf16 (+pad)

enum Act { kBF16 = 0, kF32Split = 1 };

__device__ __forceinline__ f32x4 mfma_bf16(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

// 8 bf16 (x0..x7) as four dwords (x0,x1)..(x6,x7) -> (x0,x4),(x1,x5),(x2,x6),(x3,x7)
__device__ __forceinline__ u32x4 pair_permute(u32x4 v) {
    u32x4 o;
    o.x = (v.x & 0xFFFFu) | (v.z << 16);
    o.y = (v.x >> 16) | (v.z & 0xFFFF0000u);
    o.z = (v.y & 0xFFFFu) | (v.w << 16);
    o.w = (v.y >> 16) | (v.w & 0xFFFF0000u);
    return o;
}

// packed dword of 8 nibbles (k..k+7) -> bf16 of 136+q in slot order k, k+4, k+1, k+5, ...
__device__ __forceinline__ u32x4 unpack_w4(uint32_t w) {
    w ^= 0x88888888u;
    u32x4 o;
    o.x = (w & 0x000F000Fu) | 0x43004300u;
    o.y = ((w >> 4) & 0x000F000Fu) | 0x43004300u;
    o.z = ((w >> 8) & 0x000F000Fu) | 0x43004300u;
    o.w = ((w >> 12) & 0x000F000Fu) | 0x43004300u;
    return o;
}

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// f32 -> bf16 bits, round to nearest even (finite inputs)
__device__ __forceinline__ uint32_t bf16_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// sum over the 16 lanes of a DPP row (lanes 16r .. 16r+15)
__device__ __forceinline__ float row16_sum(float v) { return lane_group_sum<16>(v); }

// One block computes a 128 (weight rows) x kBM (tokens) tile of
//   out[m, n] = sum_g s[n, g] * (sum_{k in g} (136 + q[n, k]) * a[m, k] - 136 * A_g[m])
// Gate/up mode: rows 0..63 of the tile are gate rows f0..f0+63, rows 64..127
// the up rows of the same f; the epilogue writes h = SiLU(gate) * up.
template <int kAct, bool kGateUp, int kBM>
__global__ __launch_bounds__(kBlock, kBM == 128 ? 1 : 2) void k_gemm_w4(const void* __restrict__ act,
                                                       const uint8_t* __restrict__ p0,
                                                       const uint16_t* __restrict__ s0,
                                                       const uint8_t* __restrict__ p1,
                                                       const uint16_t* __restrict__ s1,
                                                       const float* __restrict__ bias, int64_t m,
                                                       int64_t n, int64_t k,
                                                       float* __restrict__ out, int64_t out_n) {
    constexpr int kSplit = (kAct == kF32Split) ? 2 : 1;
    constexpr int kTM = kBM / 32;            // 16-token MFMA tiles per wave
    constexpr int kChunks = kBM * 16 / kBlock;  // 8-element activation blocks per thread per group
    __shared__ __attribute__((aligned(16))) uint8_t lds_w[kTileN * kWRow];
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[kSplit * kBM * kARow];
    __shared__ __attribute__((aligned(16))) uint16_t lds_s[kTileN];
    __shared__ float lds_x[kBM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wn = wave >> 1, wm = wave & 1;
    const int64_t tiles_m = (m + kBM - 1) / kBM;
    const int64_t tn = blockIdx.x / tiles_m, tmi = blockIdx.x % tiles_m;
    const int64_t m0 = tmi * kBM;
    const int64_t groups = k >> 7;
    const int64_t row_bytes = k >> 1;
    // tile row r -> weight row (gate/up: f index) and matrix
    const int64_t n0 = kGateUp ? tn * 64 : tn * kTileN;

    // ---- staging assignments ----
    // weights: thread t moves 16 B of rows (t/4) and (t/4 + 64), column 16*(t%4)
    const int wrow = tid >> 2, wcol = (tid & 3) * 16;
    // activations: block b = t + 256*i of the kBM x 16 grid of 8-element blocks
    u32x4 pw[2];
    u32x4 pa[kChunks];          // bf16: 8 bf16; split: hi half of 8 values
    u32x4 pl[kSplit == 2 ? kChunks : 1];
    float pxs[kChunks];
    uint16_t ps = 0;

    auto w_ptr = [&](int r, int64_t g) -> const uint8_t* {
        if (kGateUp) {
            const uint8_t* base = r < 64 ? p0 : p1;
            return base + (n0 + (r & 63)) * row_bytes + g * 64;
        }
        return p0 + (n0 + r) * row_bytes + g * 64;
    };
    auto w_row_valid = [&](int r) -> bool { return kGateUp ? (n0 + (r & 63)) < n : (n0 + r) < n; };

    auto load_stage = [&](int64_t g) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = wrow + 64 * i;
            pw[i] = w_row_valid(r) ? *reinterpret_cast<const u32x4*>(w_ptr(r, g) + wcol)
                                   : u32x4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
        }
        if (tid < kTileN) {
            const int r = tid;
            if (w_row_valid(r)) {
                const uint16_t* sb = kGateUp ? (r < 64 ? s0 : s1) : s0;
                ps = sb[(n0 + (kGateUp ? (r & 63) : r)) * groups + g];
            } else {
                ps = 0;
            }
        }
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int b = tid + kBlock * i;
            const int row = b >> 4, blk = b & 15;
            const int64_t mm = m0 + row;
            float part = 0.0f;
            if (kAct == kBF16) {
                u32x4 v = u32x4{0u, 0u, 0u, 0u};
                if (mm < m)
                    v = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(act) + mm * k + g * 128 +
                                                        blk * 8);
                part = bf16_lo(v.x) + bf16_hi(v.x) + bf16_lo(v.y) + bf16_hi(v.y) + bf16_lo(v.z) + bf16_hi(v.z) +
                       bf16_lo(v.w) + bf16_hi(v.w);
                pa[i] = pair_permute(v);
            } else {
                f32x4 lo4 = f32x4{0.f, 0.f, 0.f, 0.f}, hi4 = lo4;
                if (mm < m) {
                    const float* src = static_cast<const float*>(act) + mm * k + g * 128 + blk * 8;
                    lo4 = *reinterpret_cast<const f32x4*>(src);
                    hi4 = *reinterpret_cast<const f32x4*>(src + 4);
                }
                const float xv[8] = {lo4.x, lo4.y, lo4.z, lo4.w, hi4.x, hi4.y, hi4.z, hi4.w};
                uint32_t hb[8], lb[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    hb[e] = bf16_rne(xv[e]);
                    const float hf = __uint_as_float(hb[e] << 16);
                    lb[e] = bf16_rne(xv[e] - hf);
                    part += hf + __uint_as_float(lb[e] << 16);
                }
                // slot order k, k+4, k+1, k+5, k+2, k+6, k+3, k+7
                pa[i] = u32x4{hb[0] | (hb[4] << 16), hb[1] | (hb[5] << 16), hb[2] | (hb[6] << 16),
                              hb[3] | (hb[7] << 16)};
                if constexpr (kSplit == 2)
                    pl[i] = u32x4{lb[0] | (lb[4] << 16), lb[1] | (lb[5] << 16), lb[2] | (lb[6] << 16),
                                  lb[3] | (lb[7] << 16)};
            }
            pxs[i] = row16_sum(part);  // the 16 blocks of a row sit in one 16-lane DPP row
        }
    };
    auto store_stage = [&]() {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            *reinterpret_cast<u32x4*>(lds_w + (wrow + 64 * i) * kWRow + wcol) = pw[i];
        if (tid < kTileN) lds_s[tid] = ps;
#pragma unroll
        for (int i = 0; i < kChunks; ++i) {
            const int b = tid + kBlock * i;
            const int row = b >> 4, blk = b & 15;
            *reinterpret_cast<u32x4*>(lds_a + row * kARow + blk * 16) = pa[i];
            if constexpr (kSplit == 2)
                *reinterpret_cast<u32x4*>(lds_a + (kBM + row) * kARow + blk * 16) = pl[i];
            if (blk == 0) lds_x[row] = pxs[i] * 136.0f;
        }
    };

    f32x4 acc[4][kTM];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kTM; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    load_stage(0);
    store_stage();
    __syncthreads();

    const int op_row = lane & 15, op_grp = lane >> 4;
    for (int64_t g = 0; g < groups; ++g) {
        if (g + 1 < groups) load_stage(g + 1);
        f32x4 t[4][kTM];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            u32x4 a[4], b[kTM], bl[kSplit == 2 ? kTM : 1];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                a[i] = unpack_w4(*reinterpret_cast<const uint32_t*>(lds_w + (wn * 64 + i * 16 + op_row) * kWRow +
                                                                    ks * 16 + op_grp * 4));
#pragma unroll
            for (int j = 0; j < kTM; ++j) {
                const int row = wm * (kBM / 2) + j * 16 + op_row;
                b[j] = *reinterpret_cast<const u32x4*>(lds_a + row * kARow + ks * 64 + op_grp * 16);
                if constexpr (kSplit == 2)
                    bl[j] = *reinterpret_cast<const u32x4*>(lds_a + (kBM + row) * kARow + ks * 64 + op_grp * 16);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kTM; ++j) {
                    f32x4 c = (ks == 0) ? f32x4{0.f, 0.f, 0.f, 0.f} : t[i][j];
                    c = mfma_bf16(a[i], b[j], c);
                    if constexpr (kSplit == 2) c = mfma_bf16(a[i], bl[j], c);
                    t[i][j] = c;
                }
        }
        // fold the group: acc += s * (T - 136 * X)
        float xs[kTM];
#pragma unroll
        for (int j = 0; j < kTM; ++j) xs[j] = lds_x[wm * (kBM / 2) + j * 16 + op_row];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint2 sv2 = *reinterpret_cast<const uint2*>(lds_s + wn * 64 + i * 16 + op_grp * 4);
            const float sv[4] = {__half2float(__ushort_as_half(static_cast<uint16_t>(sv2.x & 0xFFFF))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(sv2.x >> 16))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(sv2.y & 0xFFFF))),
                                 __half2float(__ushort_as_half(static_cast<uint16_t>(sv2.y >> 16)))};
#pragma unroll
            for (int j = 0; j < kTM; ++j) {
                acc[i][j].x = fmaf(sv[0], t[i][j].x - xs[j], acc[i][j].x);
                acc[i][j].y = fmaf(sv[1], t[i][j].y - xs[j], acc[i][j].y);
                acc[i][j].z = fmaf(sv[2], t[i][j].z - xs[j], acc[i][j].z);
                acc[i][j].w = fmaf(sv[3], t[i][j].w - xs[j], acc[i][j].w);
            }
        }
        __syncthreads();
        if (g + 1 < groups) {
            store_stage();
            __syncthreads();
        }
    }

    // ---- epilogue: lane holds rows 4*(l/16)+r (consecutive n) of token l%16 ----
    if constexpr (!kGateUp) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int64_t nb = n0 + wn * 64 + i * 16 + op_grp * 4;
            if (nb >= n) continue;
            f32x4 bv = f32x4{0.f, 0.f, 0.f, 0.f};
            if (bias) bv = *reinterpret_cast<const f32x4*>(bias + nb);
#pragma unroll
            for (int j = 0; j < kTM; ++j) {
                const int64_t mm = m0 + wm * (kBM / 2) + j * 16 + op_row;
                if (mm < m) *reinterpret_cast<f32x4*>(out + mm * out_n + nb) = acc[i][j] + bv;
            }
        }
    } else {
        // gate waves (wn == 0) hand their tile to the up waves through LDS
        float* xg = reinterpret_cast<float*>(lds_a);  // [kBM tokens][64 f]
        if (wn == 0) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kTM; ++j) {
                    const int tok = wm * (kBM / 2) + j * 16 + op_row;
                    *reinterpret_cast<f32x4*>(xg + tok * 64 + i * 16 + op_grp * 4) = acc[i][j];
                }
        }
        __syncthreads();
        if (wn == 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t fb = n0 + i * 16 + op_grp * 4;
                if (fb >= n) continue;
#pragma unroll
                for (int j = 0; j < kTM; ++j) {
                    const int tok = wm * (kBM / 2) + j * 16 + op_row;
                    const int64_t mm = m0 + tok;
                    if (mm >= m) continue;
                    const f32x4 gv = *reinterpret_cast<const f32x4*>(xg + tok * 64 + i * 16 + op_grp * 4);
                    const f32x4 uv = acc[i][j];
                    f32x4 h;
                    h.x = gv.x * (1.0f / (1.0f + __expf(-gv.x))) * uv.x;
                    h.y = gv.y * (1.0f / (1.0f + __expf(-gv.y))) * uv.y;
                    h.z = gv.z * (1.0f / (1.0f + __expf(-gv.z))) * uv.z;
                    h.w = gv.w * (1.0f / (1.0f + __expf(-gv.w))) * uv.w;
                    *reinterpret_cast<f32x4*>(out + mm * out_n + fb) = h;
                }
            }
        }
    }
}

template <int kAct, bool kGateUp, int kBM>
int launch_w4(const void* act, const uint8_t* p0, const uint16_t* s0, const uint8_t* p1,
              const uint16_t* s1, const float* bias, int64_t m, int64_t n, int64_t k, float* out,
              int64_t out_n, hipStream_t st, const char* what) {
    const int64_t rows_per_tile = kGateUp ? 64 : kTileN;
    const int64_t tiles = ((n + rows_per_tile - 1) / rows_per_tile) * ((m + kBM - 1) / kBM);
    TQ_REQUIRE(tiles < (int64_t(1) << 31), "%s: problem too large", what);
    k_gemm_w4<kAct, kGateUp, kBM><<<static_cast<unsigned>(tiles), kBlock, 0, st>>>(act, p0, s0, p1, s1, bias, m, n, k,
                                                                                 out, out_n);
    return check_launch(what);
}

}  // namespace

// Shape-general FFN (any M; D, F multiples of 128): gate/up then down on the
// 16x16x32 kernels above, h kept as f32 [M, F] in `h`.
int launch_mlp_w4g128_general(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f, const uint8_t* gate_packed,
                              const uint16_t* gate_s, const uint8_t* up_packed, const uint16_t* up_s,
                              const uint8_t* down_packed, const uint16_t* down_s, float* h, float* y,
                              hipStream_t st) {
    int rc = launch_w4<kBF16, true, 128>(x_bf16, gate_packed, gate_s, up_packed, up_s, nullptr, m, f, d, h, f, st,
                                         "tq_mlp_w4g128 (gate/up)");
    if (rc != TQ_OK) return rc;
    return launch_w4<kF32Split, false, 64>(h, down_packed, down_s, nullptr, nullptr, nullptr, m, d, f, y, d, st,
                                           "tq_mlp_w4g128 (down)");
}

}  // namespace tq

using namespace tq;

extern "C" {

int tq_gemm_w4g128_bf16(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                        const uint16_t* s_f16, const float* bias, int64_t n, int64_t k, float* y,
                        tq_stream_t stream) {
    TQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, "tq_gemm_w4g128_bf16: negative shape");
    TQ_REQUIRE(k % 128 == 0, "tq_gemm_w4g128_bf16: K=%lld is not a multiple of 128", (long long)k);
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(y && (k == 0 || (x_bf16 && packed && s_f16)), "tq_gemm_w4g128_bf16: null pointer");
    TQ_REQUIRE(aligned(x_bf16, 2) && aligned(s_f16, 2) && aligned(y, 4) && (!bias || aligned(bias, 4)),
               "tq_gemm_w4g128_bf16: misaligned pointer");
    // the MFMA kernel tiles N by 16 rows and moves 16-byte vectors
    if (k == 0 || n % 16 != 0 || !aligned(x_bf16, 16) || !aligned(packed, 16) || !aligned(y, 16) ||
        (bias && !aligned(bias, 16)))
        return launch_linear_w4_generic(x_bf16, m, packed, s_f16, bias, n, k, y, as_hip(stream));
    return launch_w4<kBF16, false, 128>(x_bf16, packed, s_f16, nullptr, nullptr, bias, m, n, k, y, n,
                                        as_hip(stream), "tq_gemm_w4g128_bf16");
}

}  // extern "C"
