// tq_peaks.hip -- measurement kernels for bench.py (libtq_peaks.so): the
// roofline denominators re-measured on the device the bench runs on.  Not part
// of the library's C ABI; nothing in libtq.so depends on them.
//
//  * tqp_hbm_read: streams a buffer once with 16-byte nontemporal loads
//    (grid-stride, 8 loads in flight per lane) and folds it to one word per
//    block, so no load is dead.  Bytes / time over a buffer far larger than
//    the 256 MB MALL is the sustainable HBM read rate.
//  * tqp_hbm_read_chunks: the same read as one pass of blocks that each issue
//    all their loads at once (no loop), for a single read of a few tens of MB.
//  * tqp_mfma_i8 / tqp_mfma_bf16: every wave runs `iters` rounds of 8
//    independent v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_bf16 on register
//    operands (no memory traffic), one 256-thread block per CU per round of
//    blocks; ops / time is the sustained dense matrix-core rate.  The plain
//    forms use constant operands; the _random forms give every lane and chain
//    its own pseudo-random operands (i8: any code; bf16: random sign and
//    mantissa, magnitudes in [1/4, 4)), which switch the matrix cores as real
//    data does: they draw more power and the part holds a lower clock.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void k_hbm_read(const u32x4* __restrict__ p, int64_t n16, uint32_t* __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 256;
    u32x4 acc = u32x4{0, 0, 0, 0};
    int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    for (; i + 7 * stride < n16; i += 8 * stride) {
        u32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u];
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(p + i);
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o, 64);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// One pass, no loop: block b reads the 256 * 16 * kU bytes at b * that, every
// load issued before the first is consumed (the most bytes in flight a block
// can hold without a loop).
template <int kU>
__global__ __launch_bounds__(256) void k_hbm_read_chunk(const u32x4* __restrict__ p, int64_t n16,
                                                        uint32_t* __restrict__ out) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * 256 * kU + threadIdx.x;
    u32x4 v[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
        const int64_t i = base + u * 256;
        v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : u32x4{0, 0, 0, 0};
    }
    u32x4 acc = v[0];
#pragma unroll
    for (int u = 1; u < kU; ++u) acc ^= v[u];
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o, 64);
    __shared__ uint32_t part[4];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = r;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

__global__ __launch_bounds__(256, 1) void k_mfma_i8(int iters, int32_t seed, int32_t* __restrict__ out) {
    const i32x4 a = i32x4{seed + static_cast<int>(threadIdx.x), 1, 2, 3};
    const i32x4 b = i32x4{3, seed, 1, static_cast<int>(threadIdx.x)};
    i32x16 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = i32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c[j], 0, 0, 0);
    }
    int32_t r = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) r += c[j][e];
    out[blockIdx.x * 256 + threadIdx.x] = r;
}

__device__ __forceinline__ uint32_t mix(uint32_t x) {
    x ^= x >> 16;
    x *= 0x7feb352dU;
    x ^= x >> 15;
    x *= 0x846ca68bU;
    x ^= x >> 16;
    return x;
}
// two bf16 of random sign and mantissa with exponents 2^-2 .. 2^1
__device__ __forceinline__ uint32_t rnd_bf16_pair(uint32_t h) {
    const uint32_t lo = (h & 0x807Fu) | ((0x7Du + ((h >> 7) & 3u)) << 7);
    const uint32_t hi = ((h >> 16) & 0x807Fu) | ((0x7Du + ((h >> 23) & 3u)) << 7);
    return lo | (hi << 16);
}

template <bool kBf16>
__device__ __forceinline__ void random_operands(int32_t seed, u32x4 (&a)[8], u32x4 (&b)[8]) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t h = mix(threadIdx.x * 977u + blockIdx.x * 131071u + j * 7919u + static_cast<uint32_t>(seed));
        uint32_t r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = kBf16 ? rnd_bf16_pair(mix(h + e + 1)) : mix(h + e + 1);
        a[j] = u32x4{r[0], r[1], r[2], r[3]};
        b[j] = u32x4{r[4], r[5], r[6], r[7]};
    }
}

__global__ __launch_bounds__(256, 1) void k_mfma_i8_random(int iters, int32_t seed, int32_t* __restrict__ out) {
    u32x4 a[8], b[8];
    random_operands<false>(seed, a, b);
    i32x16 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = i32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, a[j]),
                                                         __builtin_bit_cast(i32x4, b[(j + 1) & 7]), c[j], 0, 0, 0);
    }
    int32_t r = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) r += c[j][e];
    out[blockIdx.x * 256 + threadIdx.x] = r;
}

__global__ __launch_bounds__(256, 1) void k_mfma_bf16_random(int iters, int32_t seed, float* __restrict__ out) {
    u32x4 a[8], b[8];
    random_operands<true>(seed, a, b);
    f32x16 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j)
            c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[j]),
                                                           __builtin_bit_cast(bf16x8, b[(j + 1) & 7]), c[j], 0, 0, 0);
    }
    float r = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) r += c[j][e];
    out[blockIdx.x * 256 + threadIdx.x] = r;
}

__global__ __launch_bounds__(256, 1) void k_mfma_bf16(int iters, float seed, float* __restrict__ out) {
    const __bf16 s = static_cast<__bf16>(seed);
    const bf16x8 a = bf16x8{s, s, s, s, s, s, s, s};
    const bf16x8 b = a;
    f32x16 c[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) c[j] = f32x16{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
    }
    float r = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e) r += c[j][e];
    out[blockIdx.x * 256 + threadIdx.x] = r;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from `buf`; `out` receives one word per block
// (blocks entries).  Returns a hipError_t.
int tqp_hbm_read(const void* buf, int64_t bytes, uint32_t* out, int blocks, hipStream_t stream) {
    k_hbm_read<<<blocks, 256, 0, stream>>>(static_cast<const u32x4*>(buf), bytes / 16, out);
    return static_cast<int>(hipGetLastError());
}

// Reads `bytes` once, each 256-thread block one contiguous run of 4096 * loads
// bytes (loads in {4, 8, 16} 16-byte loads per lane, all in flight together);
// `out` needs one word per block.
int tqp_hbm_read_chunks(const void* buf, int64_t bytes, uint32_t* out, int loads, hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    const int64_t per = 256LL * loads;
    const unsigned blocks = static_cast<unsigned>((n16 + per - 1) / per);
    const u32x4* p = static_cast<const u32x4*>(buf);
    if (loads == 4) k_hbm_read_chunk<4><<<blocks, 256, 0, stream>>>(p, n16, out);
    else if (loads == 8) k_hbm_read_chunk<8><<<blocks, 256, 0, stream>>>(p, n16, out);
    else k_hbm_read_chunk<16><<<blocks, 256, 0, stream>>>(p, n16, out);
    return static_cast<int>(hipGetLastError());
}

// `blocks` blocks of 4 waves, each wave 8 * iters MFMAs of 32x32x32 (i8: 65,536
// ops each; bf16 32x32x16: 32,768 flops each).  `out` holds blocks * 256 words.
int tqp_mfma_i8(int blocks, int iters, int32_t* out, hipStream_t stream) {
    k_mfma_i8<<<blocks, 256, 0, stream>>>(iters, 1, out);
    return static_cast<int>(hipGetLastError());
}

int tqp_mfma_bf16(int blocks, int iters, float* out, hipStream_t stream) {
    k_mfma_bf16<<<blocks, 256, 0, stream>>>(iters, 1.0f, out);
    return static_cast<int>(hipGetLastError());
}

// The same loops on pseudo-random operands (see the header).
int tqp_mfma_i8_random(int blocks, int iters, int32_t* out, hipStream_t stream) {
    k_mfma_i8_random<<<blocks, 256, 0, stream>>>(iters, 1, out);
    return static_cast<int>(hipGetLastError());
}

int tqp_mfma_bf16_random(int blocks, int iters, float* out, hipStream_t stream) {
    k_mfma_bf16_random<<<blocks, 256, 0, stream>>>(iters, 1, out);
    return static_cast<int>(hipGetLastError());
}

}  // extern "C"
