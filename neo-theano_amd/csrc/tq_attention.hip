// tq_attention.hip -- the attention core of MultiheadAttention::forward_with_mask
// (crates/theano-nn/src/transformer.rs:95-142) on gfx950, for the quantized
// q/k/v/out projections around it:
//
//   scores = (Q_h K_h^T) * (1 / sqrt(head_dim))       (+ mask, broadcast over heads)
//   P      = softmax(scores, -1)                       (tensor_ops.rs:574-620)
//   O_h    = P V_h,   heads concatenated along the embedding
//
// f32 throughout.  Q, K and V are row-major [B*S, ld] matrices whose head h
// occupies columns [h*D, (h+1)*D) (the fused QKV projection's output is read in
// place with ld = 3E); O is [B*S, ldo].
//
// One block per (128 queries, head, batch): 4 waves of 32 query rows on the
// f32 matrix cores (v_mfma_f32_32x32x2_f32).  Keys run in tiles of 32, staged
// in LDS for the 4 waves (K row-major, V transposed; both padded against bank
// conflicts), the next tile's loads in flight during the current tile's work.
// Per tile a wave computes S^T = K Q^T (lane = query, registers = keys, so the
// softmax of a query row is in-lane plus one partner lane), updates its
// running max / sum, and accumulates O^T += V^T P^T with the probabilities as
// they came out of the first product.  The head dimension is padded with zeros
// to 32, 64 or 128.  A running max of -inf (every key so far masked) leaves the
// row untouched; a row masked everywhere ends as 0/0 = NaN, as the
// reference's softmax gives.
#include <cmath>

#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kWaves = 4;
constexpr int kQW = 32;              // query rows per wave
constexpr int kQB = kWaves * kQW;    // per block
constexpr int kKT = 32;              // keys per tile
constexpr int kMaxD = 128;

__device__ __forceinline__ f32x16 mfma_f32(float a, float b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

template <int kDP>
__global__ __launch_bounds__(kWaves * kWave) void k_attention(const float* __restrict__ q, int64_t ldq,
                                                              const float* __restrict__ k, int64_t ldk,
                                                              const float* __restrict__ v, int64_t ldv,
                                                              const float* __restrict__ mask, int64_t mask_batch,
                                                              int S, int D, float scale, float* __restrict__ o,
                                                              int64_t ldo) {
    constexpr int kHalf = kDP / 2;     // d positions per lane group in S^T = K Q^T
    constexpr int kKRow = kDP + 4;     // K tile row (floats), padded
    constexpr int kVRow = kKT + 4;     // transposed V tile row, padded
    constexpr int kBlocks = kDP / 32;  // 32-wide d blocks of O^T
    constexpr int kElems = kKT * kDP / (kWaves * kWave);  // tile elements per thread (K and V each)
    __shared__ __attribute__((aligned(16))) float ks[2][kKT * kKRow];
    __shared__ __attribute__((aligned(16))) float vs[2][kDP * kVRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, g = lane >> 5, lr = lane & 31;
    const int h = blockIdx.y, b = blockIdx.z;
    const int qrow = blockIdx.x * kQB + wave * kQW + lr;  // this lane's query row
    const int64_t base = static_cast<int64_t>(b) * S;
    const int col = h * D;

    // Q fragment: d = g * kHalf + t (rows past S read row S-1; never stored)
    float qf[kHalf];
    {
        const float* qr = q + (base + min(qrow, S - 1)) * ldq + col;
#pragma unroll
        for (int t = 0; t < kHalf; ++t) {
            const int d = g * kHalf + t;
            qf[t] = d < D ? qr[d] : 0.f;
        }
    }
    const float* mrow =
        mask ? mask + ((mask_batch == 1 ? 0 : static_cast<int64_t>(b)) * S + min(qrow, S - 1)) * static_cast<int64_t>(S)
             : nullptr;

    // tile loads: element e = tid + 256 i -> key e / kDP, d e % kDP (coalesced along d)
    float kreg[kElems], vreg[kElems];
    auto load_tile = [&](int j0) {
#pragma unroll
        for (int i = 0; i < kElems; ++i) {
            const int e = tid + i * kWaves * kWave, key = e / kDP, d = e % kDP;
            const bool ok = j0 + key < S && d < D;
            const int64_t row = base + (ok ? j0 + key : 0);
            kreg[i] = ok ? k[row * ldk + col + d] : 0.f;
            vreg[i] = ok ? v[row * ldv + col + d] : 0.f;
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < kElems; ++i) {
            const int e = tid + i * kWaves * kWave, key = e / kDP, d = e % kDP;
            ks[buf][key * kKRow + d] = kreg[i];
            vs[buf][d * kVRow + key] = vreg[i];
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
        const float* kr = &ks[buf][lr * kKRow + g * kHalf];
#pragma unroll
        for (int t = 0; t < kHalf; t += 4) {
            const f32x4 kv = *reinterpret_cast<const f32x4*>(kr + t);
            st = mfma_f32(kv.x, qf[t], st);
            st = mfma_f32(kv.y, qf[t + 1], st);
            st = mfma_f32(kv.z, qf[t + 2], st);
            st = mfma_f32(kv.w, qf[t + 3], st);
        }
        float p[16];
        float mt = -INFINITY;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int key = j0 + 8 * (r >> 2) + 4 * g + (r & 3);
            float sc = st[r] * scale;
            if (key < S) {
                if (mrow) sc += mrow[key];
            } else {
                sc = -INFINITY;
            }
            p[r] = sc;
            mt = fmaxf(mt, sc);
        }
        mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));  // the partner lane holds the other 16 keys
        const float mn = fmaxf(m, mt);
        const float base_m = mn == -INFINITY ? 0.f : mn;  // all masked so far: nothing to add
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            p[r] = expf(p[r] - base_m);
            ls += p[r];
        }
        ls += __shfl_xor(ls, 32, kWave);
        const float alpha = expf(m - base_m);
        l = l * alpha + ls;
        m = mn;
        // O^T[d][q] += sum_key V[key][d] P[q][key]; step t of a 4-key run uses key 8a + 4g + b
#pragma unroll
        for (int c = 0; c < kBlocks; ++c) {
            ot[c] *= alpha;
            const float* vr = &vs[buf][(32 * c + lr) * kVRow + 4 * g];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const f32x4 vv = *reinterpret_cast<const f32x4*>(vr + 8 * a);
                ot[c] = mfma_f32(vv.x, p[4 * a + 0], ot[c]);
                ot[c] = mfma_f32(vv.y, p[4 * a + 1], ot[c]);
                ot[c] = mfma_f32(vv.z, p[4 * a + 2], ot[c]);
                ot[c] = mfma_f32(vv.w, p[4 * a + 3], ot[c]);
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
    const dim3 grid(static_cast<unsigned>((seq + kQB - 1) / kQB), static_cast<unsigned>(heads),
                    static_cast<unsigned>(batch));
    const float scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(head_dim)));
    const float* mk = mask_batch ? mask : nullptr;
    const int S = static_cast<int>(seq), D = static_cast<int>(head_dim);
    if (head_dim <= 32)
        k_attention<32><<<grid, kWaves * kWave, 0, as_hip(stream)>>>(q, ldq, k, ldk, v, ldv, mk, mask_batch, S, D,
                                                                      scale, out, ldo);
    else if (head_dim <= 64)
        k_attention<64><<<grid, kWaves * kWave, 0, as_hip(stream)>>>(q, ldq, k, ldk, v, ldv, mk, mask_batch, S, D,
                                                                      scale, out, ldo);
    else
        k_attention<128><<<grid, kWaves * kWave, 0, as_hip(stream)>>>(q, ldq, k, ldk, v, ldv, mk, mask_batch, S, D,
                                                                       scale, out, ldo);
    return check_launch("tq_attention_f32");
}
