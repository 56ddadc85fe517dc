// tq_attention.hip -- the attention core of MultiheadAttention::forward_with_mask
// (crates/theano-nn/src/transformer.rs:95-142) on gfx950, for the quantized
// q/k/v/out projections around it:
//
//   scores = (Q_h K_h^T) * (1 / sqrt(head_dim))       (+ mask, broadcast over heads)
//   P      = softmax(scores, -1)                       (tensor_ops.rs:574-620)
//   O_h    = P V_h,   heads concatenated along the embedding
//
// f32 inputs, outputs, softmax and accumulators.  Q, K and V are row-major [B*S, ld] matrices whose head h
// occupies columns [h*D, (h+1)*D) (the fused QKV projection's output is read in
// place with ld = 3E); O is [B*S, ldo].
//
// One block per (128 queries, head, batch): 4 waves of 32 query rows on the
// bf16 matrix cores (v_mfma_f32_32x32x16_bf16).  Every f32 operand is split
// exactly into bf16 hi = bf16(v) and lo = bf16(v - hi) (|v - hi - lo| <=
// 2^-18 |v|), and each product runs as hi*hi + hi*lo + lo*hi, all bf16 products
// exact in the f32 accumulators; the dropped lo*lo term is below 2^-16 of the
// product.  Keys run in tiles of 32, staged in LDS for the 4 waves as hi and lo
// planes (K row-major, V transposed, both padded against bank conflicts), the
// next tile's loads in flight during the current tile's work.  Scores are kept
// in log2 units (scale * log2(e), the mask likewise), so each probability is
// one v_exp_f32 (2^x).  Per tile a wave computes S^T = K Q^T (lane = query, registers = keys, so the softmax of a
// query row is in-lane plus one partner lane), updates its running max / sum,
// and accumulates O^T += V^T P^T with the probabilities as they came out of the
// first product: lane half g holds keys 8a + 4g + b (a, b < 4), and the
// transposed V tile stores key k at column k with bits 2 and 3 swapped, so the
// 8 keys of a 16-key MFMA step are one contiguous 16-byte read.  The head
// dimension is padded with zeros to 32, 64 or 128.  A running max of -inf
// (every key so far masked) leaves the row untouched; a row masked everywhere
// ends as 0/0 = NaN, as the reference's softmax gives.
//
// With D % 4 == 0 and 16-byte aligned K and V rows (k_attention_vec) a thread
// loads K as 16-byte quads along d and V as four keys at one d (coalesced
// along d across the wave), both stored to LDS as 8-byte runs, with offsets
// fixed per thread and a uniform step per item, so whole tiles load without
// clamps; it fits two waves per SIMD in 256 registers.  Other head dimensions
// keep the per-element loads (k_attention, one wave per SIMD).  At head dim 128
// a launch with a block per CU or more takes 8-wave blocks (256 queries, each
// key tile loaded and split once for all of them).  All forms give the same
// bits.
#include <cmath>

#include "tq_internal.h"

namespace tq {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kWaves = 4;           // waves per block (8 in the wide form)
constexpr int kQW = 32;              // query rows per wave
constexpr int kKT = 32;              // keys per tile
constexpr int kMaxD = 128;

__device__ __forceinline__ f32x16 mfma_bf16(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ uint16_t bf16_bits(float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); }
__device__ __forceinline__ float bf16_value(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// v = hi + lo (+ < 2^-18 |v|): hi = bf16(v), lo = bf16(v - hi)
__device__ __forceinline__ void split(float v, uint16_t& hi, uint16_t& lo) {
    hi = bf16_bits(v);
    lo = bf16_bits(v - bf16_value(hi));
}

// 8 f32 -> packed bf16 hi and lo
__device__ __forceinline__ void split8(const float* v, u32x4& hi, u32x4& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint16_t h0, l0, h1, l1;
        split(v[2 * i], h0, l0);
        split(v[2 * i + 1], h1, l1);
        h[i] = h0 | static_cast<uint32_t>(h1) << 16;
        l[i] = l0 | static_cast<uint32_t>(l1) << 16;
    }
    hi = u32x4{h[0], h[1], h[2], h[3]};
    lo = u32x4{l[0], l[1], l[2], l[3]};
}

__device__ __forceinline__ int vcol(int key) { return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1); }

// kVec: D % 4 == 0 and 16-byte aligned rows of K and V, loaded as whole quads.
// kW waves per block share each key tile (kW x 32 queries).
template <int kDP, bool kVec, int kW>
__device__ __forceinline__ void attention_block(const float* __restrict__ q, int64_t ldq,
                                                              const float* __restrict__ k, int64_t ldk,
                                                              const float* __restrict__ v, int64_t ldv,
                                                              const float* __restrict__ mask, int64_t mask_batch,
                                                              int S, int D, float scale, float* __restrict__ o,
                                                              int64_t ldo) {
    constexpr int kSteps = kDP / 16;   // 16-wide d steps of S^T = K Q^T
    constexpr int kKRow = kDP + 8;     // K plane row (bf16), padded
    constexpr int kVRow = kKT + 8;     // transposed V plane row (bf16), padded
    constexpr int kBlocks = kDP / 32;  // 32-wide d blocks of O^T
    constexpr int kElems = kKT * kDP / (kW * kWave);  // tile elements per thread (K and V each)
    static_assert(!kVec || kElems % 4 == 0, "whole quads per thread");
    __shared__ __attribute__((aligned(16))) uint16_t ksh[2][kKT * kKRow], ksl[2][kKT * kKRow];
    __shared__ __attribute__((aligned(16))) uint16_t vsh[2][kDP * kVRow], vsl[2][kDP * kVRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, lr = lane & 31;
    const int h = blockIdx.y, b = blockIdx.z;
    const int qrow = blockIdx.x * (kW * kQW) + wave * kQW + lr;  // this lane's query row
    const int64_t base = static_cast<int64_t>(b) * S;
    const int col = h * D;
    constexpr float kLog2e = 1.4426950408889634f;
    const float scale2 = scale * kLog2e;

    // Q operand: step s covers d = 16 s + 8 g + j (rows past S read row S-1; never stored)
    u32x4 qh[kSteps], ql[kSteps];
    {
        const float* qr = q + (base + min(qrow, S - 1)) * ldq + col;
#pragma unroll
        for (int st = 0; st < kSteps; ++st) {
            float qv[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = 16 * st + 8 * g + j;
                qv[j] = d < D ? qr[d] : 0.f;
            }
            split8(qv, qh[st], ql[st]);
        }
    }
    const float* mrow =
        mask ? mask + ((mask_batch == 1 ? 0 : static_cast<int64_t>(b)) * S + min(qrow, S - 1)) * static_cast<int64_t>(S)
             : nullptr;

    // tile loads.  Scalar: element e = tid + 256 i -> key e / kDP, d e % kDP
    // (coalesced along d).  kVec: K item e -> key e / (kDP / 4), the quad of d
    // from 4 (e % (kDP / 4)), one 16-byte load; V item e -> d = e % kDP and keys
    // 4 (e / kDP) .. + 3, four loads coalesced along d across the wave, so that
    // both land in LDS as 8-byte runs (K along d, the transposed V along keys).
    // Rows past S and d past D read clamped addresses and are zeroed.
    constexpr int kQuads = kElems / 4;  // K and V items per thread (kVec)
    float kreg[kElems], vreg[kElems];
    // kVec: the element offsets of item 0 from its tile's first row (the host
    // keeps a tile's offsets below 2^31) and whether its d is inside the head;
    // item i has the same d and keys 256 i / (kDP / 4) (K) or 4 (256 i / kDP)
    // (V) further on
    constexpr int kKeyStepK = kW * kWave / (kDP / 4), kKeyStepV = 4 * (kW * kWave / kDP);
    const int dq = 4 * (tid % (kDP / 4)), dv = tid % kDP;
    const uint32_t koff = static_cast<uint32_t>((tid / (kDP / 4)) * ldk + col + min(dq, D - 4));
    const uint32_t voff = static_cast<uint32_t>(4 * (tid / kDP) * ldv + col + min(dv, D - 1));
    const bool kin = dq < D, vin = dv < D;
    auto load_tile = [&](int j0) {
        if constexpr (kVec) {
            if (j0 + kKT <= S) {  // a whole tile (uniform): no row clamps
#pragma unroll
                for (int i = 0; i < kQuads; ++i) {
                    const float* kb = k + (base + j0 + i * kKeyStepK) * ldk;
                    const float4 kv = *reinterpret_cast<const float4*>(kb + koff);
                    kreg[4 * i] = kin ? kv.x : 0.f;
                    kreg[4 * i + 1] = kin ? kv.y : 0.f;
                    kreg[4 * i + 2] = kin ? kv.z : 0.f;
                    kreg[4 * i + 3] = kin ? kv.w : 0.f;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float x = (v + (base + j0 + i * kKeyStepV + r) * ldv)[voff];
                        vreg[4 * i + r] = vin ? x : 0.f;
                    }
                }
                return;
            }
#pragma unroll
            for (int i = 0; i < kQuads; ++i) {
                const int e = tid + i * kW * kWave;
                const int key = e / (kDP / 4), d = 4 * (e % (kDP / 4));
                const bool ok = j0 + key < S && d < D;
                const int64_t row = base + min(j0 + key, S - 1);
                const float4 kv = *reinterpret_cast<const float4*>(k + row * ldk + col + min(d, D - 4));
                kreg[4 * i] = ok ? kv.x : 0.f;
                kreg[4 * i + 1] = ok ? kv.y : 0.f;
                kreg[4 * i + 2] = ok ? kv.z : 0.f;
                kreg[4 * i + 3] = ok ? kv.w : 0.f;
                const int dv = e % kDP, k4 = 4 * (e / kDP);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool okv = j0 + k4 + r < S && dv < D;
                    const float x = v[(base + min(j0 + k4 + r, S - 1)) * ldv + col + min(dv, D - 1)];
                    vreg[4 * i + r] = okv ? x : 0.f;
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < kElems; ++i) {
                const int e = tid + i * kW * kWave, key = e / kDP, d = e % kDP;
                const bool ok = j0 + key < S && d < D;
                const int64_t row = base + (ok ? j0 + key : 0);
                kreg[i] = ok ? k[row * ldk + col + d] : 0.f;
                vreg[i] = ok ? v[row * ldv + col + d] : 0.f;
            }
        }
    };
    auto store_tile = [&](int buf) {
        if constexpr (kVec) {
#pragma unroll
            for (int i = 0; i < kQuads; ++i) {
                const int e = tid + i * kW * kWave;
                const int key = e / (kDP / 4), d = 4 * (e % (kDP / 4));
                uint16_t h4[4], l4[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) split(kreg[4 * i + r], h4[r], l4[r]);
                *reinterpret_cast<uint2*>(&ksh[buf][key * kKRow + d]) =
                    make_uint2(h4[0] | static_cast<uint32_t>(h4[1]) << 16, h4[2] | static_cast<uint32_t>(h4[3]) << 16);
                *reinterpret_cast<uint2*>(&ksl[buf][key * kKRow + d]) =
                    make_uint2(l4[0] | static_cast<uint32_t>(l4[1]) << 16, l4[2] | static_cast<uint32_t>(l4[3]) << 16);
                const int dv = e % kDP, k4 = 4 * (e / kDP);
#pragma unroll
                for (int r = 0; r < 4; ++r) split(vreg[4 * i + r], h4[r], l4[r]);
                // keys 4a .. 4a + 3 sit at 4 consecutive columns of the transposed tile
                *reinterpret_cast<uint2*>(&vsh[buf][dv * kVRow + vcol(k4)]) =
                    make_uint2(h4[0] | static_cast<uint32_t>(h4[1]) << 16, h4[2] | static_cast<uint32_t>(h4[3]) << 16);
                *reinterpret_cast<uint2*>(&vsl[buf][dv * kVRow + vcol(k4)]) =
                    make_uint2(l4[0] | static_cast<uint32_t>(l4[1]) << 16, l4[2] | static_cast<uint32_t>(l4[3]) << 16);
            }
        } else {
#pragma unroll
            for (int i = 0; i < kElems; ++i) {
                const int e = tid + i * kW * kWave, key = e / kDP, d = e % kDP;
                uint16_t hi, lo;
                split(kreg[i], hi, lo);
                ksh[buf][key * kKRow + d] = hi;
                ksl[buf][key * kKRow + d] = lo;
                split(vreg[i], hi, lo);
                vsh[buf][d * kVRow + vcol(key)] = hi;
                vsl[buf][d * kVRow + vcol(key)] = lo;
            }
        }
    };

    f32x16 ot[kBlocks];
#pragma unroll
    for (int c = 0; c < kBlocks; ++c) ot[c] = f32x16{};
    float m = -INFINITY, l = 0.f;

    load_tile(0);
    store_tile(0);
    __syncthreads();
    int buf = 0;
    for (int j0 = 0; j0 < S; j0 += kKT) {
        const bool more = j0 + kKT < S;
        if (more) load_tile(j0 + kKT);  // in flight during this tile

        // S^T[key][q] = sum_d K[key][d] Q[q][d]: lane holds keys 8(r/4) + 4g + r%4 of query lr
        f32x16 st = f32x16{};
        {
            const uint16_t* kh = &ksh[buf][lr * kKRow + 8 * g];
            const uint16_t* kl = &ksl[buf][lr * kKRow + 8 * g];
#pragma unroll
            for (int s2 = 0; s2 < kSteps; ++s2) {
                const u32x4 a_h = *reinterpret_cast<const u32x4*>(kh + 16 * s2);
                const u32x4 a_l = *reinterpret_cast<const u32x4*>(kl + 16 * s2);
                st = mfma_bf16(a_h, qh[s2], st);
                st = mfma_bf16(a_h, ql[s2], st);
                st = mfma_bf16(a_l, qh[s2], st);
            }
        }
        // scores in log2 units: s * scale * log2(e) (+ mask * log2(e)), so that the
        // probabilities are one v_exp_f32 (2^x) each
        float p[16];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = j0 + 8 * (r >> 2) + 4 * g + (r & 3);
            float sc = st[r] * scale2;
            // `mask` (a kernel argument) is uniform: no divergent branch; the index is clamped
            if (mask) sc = fmaf(mrow[min(key, S - 1)], kLog2e, sc);
            sc = key < S ? sc : -INFINITY;
            p[r] = sc;
            mt = fmaxf(mt, sc);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));  // the partner lane holds the other 16 keys
        const float mn = fmaxf(m, mt);
        const float base_m = mn == -INFINITY ? 0.f : mn;  // all masked so far: nothing to add
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = __builtin_amdgcn_exp2f(p[r] - base_m);
            ls += p[r];
        }
        ls += __shfl_xor(ls, 32, kWave);
        const float alpha = __builtin_amdgcn_exp2f(m - base_m);
        l = l * alpha + ls;
        m = mn;
        // P^T operand: step t of 16 keys takes registers 8t .. 8t+7 (keys 16t + 8h + 4g + b,
        // slot 4h + b), the order of the transposed V tile's columns
        u32x4 ph[2], pl[2];
        split8(p, ph[0], pl[0]);
        split8(p + 8, ph[1], pl[1]);
        // O^T[d][q] += sum_key V[key][d] P[q][key]
        // alpha is 1 in every lane once the running maxima settle: the rescale is skipped
        const bool rescale = __ballot(alpha != 1.0f) != 0;
#pragma unroll
        for (int c = 0; c < kBlocks; ++c) {
            if (rescale) ot[c] *= alpha;
            const uint16_t* vh = &vsh[buf][(32 * c + lr) * kVRow + 8 * g];
            const uint16_t* vl = &vsl[buf][(32 * c + lr) * kVRow + 8 * g];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const u32x4 a_h = *reinterpret_cast<const u32x4*>(vh + 16 * t);
                const u32x4 a_l = *reinterpret_cast<const u32x4*>(vl + 16 * t);
                ot[c] = mfma_bf16(a_h, ph[t], ot[c]);
                ot[c] = mfma_bf16(a_h, pl[t], ot[c]);
                ot[c] = mfma_bf16(a_l, ph[t], ot[c]);
            }
        }
        if (more) {
            store_tile(buf ^ 1);  // the other buffer: last read before the previous barrier
            __syncthreads();
            buf ^= 1;
        }
    }
    // lane holds O^T[d = 32c + 8(r/4) + 4g + r%4][q = lr]
    if (qrow < S) {
        float* orow = o + (base + qrow) * ldo + col;
        const float inv = 1.0f / l;
#pragma unroll
        for (int c = 0; c < kBlocks; ++c)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int d = 32 * c + 8 * (r >> 2) + 4 * g + (r & 3);
                if (d < D) orow[d] = ot[c][r] * inv;
            }
    }
}

// Two waves per SIMD where the quad loads leave the registers for them (256 per
// lane); the scalar form keeps one (its element loads need more).  kW = 8: the
// wide form, 256 queries per block, each key tile loaded and split once for
// twice as many queries.
template <int kDP, int kW>
__global__ __launch_bounds__(kW * kWave) __attribute__((amdgpu_waves_per_eu(2))) void k_attention_vec(
    const float* __restrict__ q, int64_t ldq, const float* __restrict__ k, int64_t ldk, const float* __restrict__ v,
    int64_t ldv, const float* __restrict__ mask, int64_t mask_batch, int S, int D, float scale, float* __restrict__ o,
    int64_t ldo) {
    attention_block<kDP, true, kW>(q, ldq, k, ldk, v, ldv, mask, mask_batch, S, D, scale, o, ldo);
}

template <int kDP>
__global__ __launch_bounds__(kWaves * kWave) void k_attention(const float* __restrict__ q, int64_t ldq,
                                                              const float* __restrict__ k, int64_t ldk,
                                                              const float* __restrict__ v, int64_t ldv,
                                                              const float* __restrict__ mask, int64_t mask_batch,
                                                              int S, int D, float scale, float* __restrict__ o,
                                                              int64_t ldo) {
    attention_block<kDP, false, kWaves>(q, ldq, k, ldk, v, ldv, mask, mask_batch, S, D, scale, o, ldo);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" int tq_attention_f32(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                                int64_t ldv, const float* mask, int64_t mask_batch, int64_t batch, int64_t seq,
                                int64_t heads, int64_t head_dim, float* out, int64_t ldo, tq_stream_t stream) {
    TQ_REQUIRE(batch >= 0 && seq >= 0 && heads >= 0 && head_dim >= 0, "tq_attention_f32: negative shape");
    if (batch == 0 || seq == 0 || heads == 0) return TQ_OK;
    TQ_REQUIRE(head_dim >= 1 && head_dim <= kMaxD, "tq_attention_f32: head_dim=%lld outside [1, %d]",
               (long long)head_dim, kMaxD);
    TQ_REQUIRE(q && k && v && out, "tq_attention_f32: null pointer");
    const int64_t e = heads * head_dim;
    TQ_REQUIRE(ldq >= e && ldk >= e && ldv >= e && ldo >= e, "tq_attention_f32: row stride below heads * head_dim");
    TQ_REQUIRE(mask_batch == 0 || mask_batch == 1 || mask_batch == batch,
               "tq_attention_f32: mask_batch must be 0 (no mask), 1 or batch");
    TQ_REQUIRE(mask_batch == 0 || mask, "tq_attention_f32: null mask");
    TQ_REQUIRE(seq < (int64_t(1) << 30) && heads < 65536 && batch < 65536, "tq_attention_f32: problem too large");
    TQ_REQUIRE(aligned(q, 4) && aligned(k, 4) && aligned(v, 4) && aligned(out, 4) && (!mask || aligned(mask, 4)),
               "tq_attention_f32: misaligned pointer");
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
    const float* mk = mask_batch ? mask : nullptr;
    const int S = static_cast<int>(seq), D = static_cast<int>(head_dim);
    // whole quads of d where every K and V row is 16-byte aligned
    // (and element offsets within a key tile below 2^31)
    const bool vec = head_dim % 4 == 0 && ldk % 4 == 0 && ldv % 4 == 0 && aligned(k, 16) && aligned(v, 16) &&
                     kKT * std::max(ldk, ldv) + e < (int64_t(1) << 31);
    // head dim 128: 8-wave blocks where they still give every CU a block (measured
    // at S = 2048, H = 32: 310-315 against 343 us eager)
    const int64_t wide_blocks = (seq + 8 * kQW - 1) / (8 * kQW) * heads * batch;
    const int waves = vec && head_dim > 64 && wide_blocks >= device_cu_count() ? 8 : kWaves;
    const dim3 grid(static_cast<unsigned>((seq + waves * kQW - 1) / (waves * kQW)), static_cast<unsigned>(heads),
                    static_cast<unsigned>(batch));
#define TQ_ATT(KERNEL, ...)                                                                                     \
    KERNEL<__VA_ARGS__><<<grid, waves * kWave, 0, as_hip(stream)>>>(q, ldq, k, ldk, v, ldv, mk, mask_batch, S, D, \
                                                                    scale, out, ldo)
    if (head_dim <= 32) {
        if (vec) TQ_ATT(k_attention_vec, 32, kWaves); else TQ_ATT(k_attention, 32);
    } else if (head_dim <= 64) {
        if (vec) TQ_ATT(k_attention_vec, 64, kWaves); else TQ_ATT(k_attention, 64);
    } else if (vec) {
        if (waves == 8) TQ_ATT(k_attention_vec, 128, 8); else TQ_ATT(k_attention_vec, 128, kWaves);
    } else {
        TQ_ATT(k_attention, 128);
    }
#undef TQ_ATT
    return check_launch("tq_attention_f32");
}
