// tq_generic.hip -- shape-general quantized Linear kernels.
//
// The tuned kernels need tile-friendly shapes (K a multiple of 16, N of 16,
// 16-byte aligned rows, K within an LDS budget).  A drop-in for the
// reference's Linear (crates/theano-nn/src/linear.rs:111-121) must take any
// shape, so every matmul entry point falls back to these kernels when its
// fast kernel's constraints are not met.  One wave computes one output
// element: lanes stride over K with element-sized loads (any alignment), a
// wave64 butterfly sums the lanes.  Results follow the same formulas as the
// fast kernels: f32 accumulation for weight-only paths, exact int32
// accumulation for W8A8.
#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kGenBlock = 256;
constexpr int kGenWaves = kGenBlock / kWave;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// y[i, j] = s[j] * sum_k x[i, k] q[j, k] + b[j]
// value of an 8-bit code: int8_t INT8, uint8_t FP8 (OCP e4m3)
__device__ __forceinline__ float code_value(int8_t c) { return static_cast<float>(c); }
__device__ __forceinline__ float code_value(uint8_t c) { return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(c), 0); }

template <class Code>
__global__ __launch_bounds__(kGenBlock) void k_linear_8bit_generic(const float* __restrict__ x, int64_t m,
                                                                   const Code* __restrict__ q,
                                                                   const float* __restrict__ s,
                                                                   const float* __restrict__ bias, int64_t n,
                                                                   int64_t k, float* __restrict__ y) {
    const int64_t out = static_cast<int64_t>(blockIdx.x) * kGenWaves + threadIdx.x / kWave;
    if (out >= m * n) return;  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t i = out / n, j = out % n;
    const float* xr = x + i * k;
    const Code* qr = q + j * k;
    float acc = 0.f;
    for (int64_t p = lane; p < k; p += kWave) acc += xr[p] * code_value(qr[p]);
    acc = wave_sum(acc);
    if (lane == 0) y[out] = acc * s[j] + (bias ? bias[j] : 0.f);
}

// y[i, j] = sum_g s[j, g] * sum_{k in g} x[i, k] q[j, k] + b[j]   (K % 128 == 0)
__global__ __launch_bounds__(kGenBlock) void k_linear_w4_generic(const uint16_t* __restrict__ x, int64_t m,
                                                                 const uint8_t* __restrict__ packed,
                                                                 const uint16_t* __restrict__ s16,
                                                                 const float* __restrict__ bias, int64_t n,
                                                                 int64_t k, float* __restrict__ y) {
    const int64_t out = static_cast<int64_t>(blockIdx.x) * kGenWaves + threadIdx.x / kWave;
    if (out >= m * n) return;  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t i = out / n, j = out % n;
    const uint16_t* xr = x + i * k;
    const uint8_t* pr = packed + j * (k / 2);
    const uint16_t* sr = s16 + j * (k / 128);
    float total = 0.f;
    for (int64_t g = 0; g < k / 128; ++g) {
        // lane covers byte g*64 + lane: elements 2 lane, 2 lane + 1 of the group
        const uint8_t b = pr[g * 64 + lane];
        const int q0 = static_cast<int>(static_cast<int8_t>(static_cast<uint8_t>(b << 4))) >> 4;
        const int q1 = static_cast<int>(static_cast<int8_t>(b)) >> 4;
        const int64_t k0 = g * 128 + 2 * lane;
        float part = bf16_to_f32(xr[k0]) * static_cast<float>(q0) + bf16_to_f32(xr[k0 + 1]) * static_cast<float>(q1);
        part = wave_sum(part);
        total += __half2float(__ushort_as_half(sr[g])) * part;
    }
    if (lane == 0) y[out] = total + (bias ? bias[j] : 0.f);
}

// acc[i, j] = sum_k qa[i, k] qw[j, k] (int32, exact); y = fma(f32(acc) * sa[i], sw[j], b[j])
__global__ __launch_bounds__(kGenBlock) void k_gemm_w8a8_generic(const int8_t* __restrict__ qa,
                                                                 const float* __restrict__ sa,
                                                                 const int8_t* __restrict__ qw,
                                                                 const float* __restrict__ sw,
                                                                 const float* __restrict__ bias, int64_t m,
                                                                 int64_t n, int64_t k,
                                                                 int32_t* __restrict__ acc_out,
                                                                 float* __restrict__ y) {
    const int64_t out = static_cast<int64_t>(blockIdx.x) * kGenWaves + threadIdx.x / kWave;
    if (out >= m * n) return;  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t i = out / n, j = out % n;
    const int8_t* ar = qa + i * k;
    const int8_t* wr = qw + j * k;
    int acc = 0;
    for (int64_t p = lane; p < k; p += kWave) acc += static_cast<int>(ar[p]) * static_cast<int>(wr[p]);
    acc = wave_sum(acc);
    if (lane == 0) {
        if (acc_out) acc_out[out] = acc;
        y[out] = fmaf(static_cast<float>(acc) * sa[i], sw[j], bias ? bias[j] : 0.f);
    }
}

// FP8 (e4m3) codes: products exact in f32, f32 sum over K, then the scales.
__global__ __launch_bounds__(kGenBlock) void k_gemm_fp8_generic(const uint8_t* __restrict__ qa,
                                                                const float* __restrict__ sa,
                                                                const uint8_t* __restrict__ qw,
                                                                const float* __restrict__ sw,
                                                                const float* __restrict__ bias, int64_t m,
                                                                int64_t n, int64_t k, float* __restrict__ y) {
    const int64_t out = static_cast<int64_t>(blockIdx.x) * kGenWaves + threadIdx.x / kWave;
    if (out >= m * n) return;  // wave-uniform
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t i = out / n, j = out % n;
    const uint8_t* ar = qa + i * k;
    const uint8_t* wr = qw + j * k;
    float acc = 0.f;
    for (int64_t p = lane; p < k; p += kWave)
        acc += code_value(ar[p]) * code_value(wr[p]);
    acc = wave_sum(acc);
    if (lane == 0) y[out] = fmaf(acc * sa[i], sw[j], bias ? bias[j] : 0.f);
}

unsigned generic_grid(int64_t outputs) { return static_cast<unsigned>((outputs + kGenWaves - 1) / kGenWaves); }

}  // namespace

int launch_linear_8bit_generic(const float* x, int64_t m, const int8_t* q, const float* s, const float* bias,
                               int64_t n, int64_t k, float* y, hipStream_t st) {
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(m * n / kGenWaves < (int64_t(1) << 31), "linear (generic): too many outputs");
    k_linear_8bit_generic<int8_t><<<generic_grid(m * n), kGenBlock, 0, st>>>(x, m, q, s, bias, n, k, y);
    return check_launch("linear_w8 (generic)");
}

int launch_linear_8bit_generic(const float* x, int64_t m, const uint8_t* q, const float* s, const float* bias,
                               int64_t n, int64_t k, float* y, hipStream_t st) {
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(m * n / kGenWaves < (int64_t(1) << 31), "linear (generic): too many outputs");
    k_linear_8bit_generic<uint8_t><<<generic_grid(m * n), kGenBlock, 0, st>>>(x, m, q, s, bias, n, k, y);
    return check_launch("linear_fp8 (generic)");
}

int launch_linear_w4_generic(const uint16_t* x, int64_t m, const uint8_t* packed, const uint16_t* s16,
                             const float* bias, int64_t n, int64_t k, float* y, hipStream_t st) {
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(m * n / kGenWaves < (int64_t(1) << 31), "linear (generic): too many outputs");
    k_linear_w4_generic<<<generic_grid(m * n), kGenBlock, 0, st>>>(x, m, packed, s16, bias, n, k, y);
    return check_launch("linear_w4g128 (generic)");
}

int launch_gemm_w8a8_generic(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                             const float* bias, int64_t m, int64_t n, int64_t k, int32_t* acc, float* y,
                             hipStream_t st) {
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(m * n / kGenWaves < (int64_t(1) << 31), "gemm_w8a8 (generic): too many outputs");
    k_gemm_w8a8_generic<<<generic_grid(m * n), kGenBlock, 0, st>>>(qa, sa, qw, sw, bias, m, n, k, acc, y);
    return check_launch("gemm_w8a8 (generic)");
}

int launch_gemm_fp8_generic(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                            const float* bias, int64_t m, int64_t n, int64_t k, float* y, hipStream_t st) {
    if (m == 0 || n == 0) return TQ_OK;
    TQ_REQUIRE(m * n / kGenWaves < (int64_t(1) << 31), "gemm_fp8 (generic): too many outputs");
    k_gemm_fp8_generic<<<generic_grid(m * n), kGenBlock, 0, st>>>(qa, sa, qw, sw, bias, m, n, k, y);
    return check_launch("gemm_fp8 (generic)");
}

}  // namespace tq
