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
// One block per (16 queries, head, batch): 4 waves of 4 query rows.  Keys run
// in tiles of 64 staged in LDS (K padded against bank conflicts); lane j
// scores key j of the tile for the wave's 4 rows (q rows broadcast from LDS),
// an online softmax keeps the running max / sum per row, and P V accumulates
// with lanes over the head dimension.  A running max of -inf (every key so far
// masked) leaves the row untouched; a row masked everywhere ends as 0/0 = NaN,
// as the reference's softmax gives.
#include <cmath>

#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kWaves = 4;
constexpr int kRowsPerWave = 4;
constexpr int kQB = kWaves * kRowsPerWave;  // queries per block
constexpr int kKT = 64;                     // keys per tile
constexpr int kMaxD = 128;

__global__ __launch_bounds__(kWaves * kWave) void k_attention(const float* __restrict__ q, int64_t ldq,
                                                              const float* __restrict__ k, int64_t ldk,
                                                              const float* __restrict__ v, int64_t ldv,
                                                              const float* __restrict__ mask, int64_t mask_batch,
                                                              int S, int D, float scale, float* __restrict__ o,
                                                              int64_t ldo) {
    __shared__ float kt[kKT][kMaxD + 1];
    __shared__ float vt[kKT][kMaxD];
    __shared__ f32x4 qs[kWaves][kMaxD];          // the wave's 4 rows, element d of each in one f32x4
    __shared__ f32x4 ps[kWaves][kKT];            // probabilities of the tile for the 4 rows
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const int i0 = blockIdx.x * kQB + wave * kRowsPerWave;  // first query row of this wave
    const int64_t rowbase = static_cast<int64_t>(b) * S;
    const int col = h * D;

    // q rows of this wave (rows past S read row S-1; never stored)
    for (int d = lane; d < D; d += kWave) {
        f32x4 t;
        t.x = q[(rowbase + min(i0 + 0, S - 1)) * ldq + col + d];
        t.y = q[(rowbase + min(i0 + 1, S - 1)) * ldq + col + d];
        t.z = q[(rowbase + min(i0 + 2, S - 1)) * ldq + col + d];
        t.w = q[(rowbase + min(i0 + 3, S - 1)) * ldq + col + d];
        qs[wave][d] = t;
    }
    const float* mrow[kRowsPerWave];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r)
        mrow[r] = mask ? mask + ((mask_batch == 1 ? 0 : static_cast<int64_t>(b)) * S + min(i0 + r, S - 1)) *
                                    static_cast<int64_t>(S)
                       : nullptr;

    float m[kRowsPerWave], l[kRowsPerWave], acc[kRowsPerWave][2];
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
        acc[r][0] = acc[r][1] = 0.f;
    }

    for (int j0 = 0; j0 < S; j0 += kKT) {
        __syncthreads();  // previous tile fully consumed
        for (int e = tid; e < kKT * D; e += kWaves * kWave) {
            const int j = e / D, d = e - j * D;
            const bool ok = j0 + j < S;
            const int64_t row = rowbase + (ok ? j0 + j : 0);
            kt[j][d] = ok ? k[row * ldk + col + d] : 0.f;
            vt[j][d] = ok ? v[row * ldv + col + d] : 0.f;
        }
        __syncthreads();
        // scores of key j0 + lane for the 4 rows
        float s[kRowsPerWave] = {0.f, 0.f, 0.f, 0.f};
        for (int d = 0; d < D; ++d) {
            const float kv = kt[lane][d];
            const f32x4 qv = qs[wave][d];
            s[0] = fmaf(qv.x, kv, s[0]);
            s[1] = fmaf(qv.y, kv, s[1]);
            s[2] = fmaf(qv.z, kv, s[2]);
            s[3] = fmaf(qv.w, kv, s[3]);
        }
        const bool kval = j0 + lane < S;
        float p[kRowsPerWave];
#pragma unroll
        for (int r = 0; r < kRowsPerWave; ++r) {
            float sc = s[r] * scale;
            if (mrow[r] && kval) sc += mrow[r][j0 + lane];
            sc = kval ? sc : -INFINITY;
            const float mt = wave_max(sc);
            const float mn = fmaxf(m[r], mt);
            const float base = mn == -INFINITY ? 0.f : mn;  // all masked so far: nothing to add
            p[r] = expf(sc - base);
            const float alpha = expf(m[r] - base);
            l[r] = l[r] * alpha + wave_sum(p[r]);
            acc[r][0] *= alpha;
            acc[r][1] *= alpha;
            m[r] = mn;
        }
        // the wave's lanes exchange p through LDS (in order within a wave)
        ps[wave][lane] = f32x4{p[0], p[1], p[2], p[3]};
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int jn = min(kKT, S - j0);
        for (int j = 0; j < jn; ++j) {
            const f32x4 pj = ps[wave][j];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int d = lane + c * kWave;
                if (d < D) {
                    const float vv = vt[j][d];
                    acc[0][c] = fmaf(pj.x, vv, acc[0][c]);
                    acc[1][c] = fmaf(pj.y, vv, acc[1][c]);
                    acc[2][c] = fmaf(pj.z, vv, acc[2][c]);
                    acc[3][c] = fmaf(pj.w, vv, acc[3][c]);
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRowsPerWave; ++r) {
        const int i = i0 + r;
        if (i >= S) continue;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int d = lane + c * kWave;
            if (d < D) o[(rowbase + i) * ldo + col + d] = acc[r][c] / l[r];
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
    k_attention<<<grid, kWaves * kWave, 0, as_hip(stream)>>>(q, ldq, k, ldk, v, ldv, mask_batch ? mask : nullptr,
                                                             mask_batch, static_cast<int>(seq),
                                                             static_cast<int>(head_dim), scale, out, ldo);
    return check_launch("tq_attention_f32");
}
