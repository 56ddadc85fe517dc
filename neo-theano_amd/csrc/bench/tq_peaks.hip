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
//  * tqp_hbm_read_waves: the same bytes in the INT4 decode GEMV's access
//    pattern (1024-thread blocks, 1 KB per wave load, a window of loads in
//    flight), without its arithmetic.
//  * tqp_mfma_i8 / tqp_mfma_bf16: every wave runs `iters` rounds of 8
//    independent v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_bf16 on register
//    operands (no memory traffic), one 256-thread block per CU per round of
//    blocks; ops / time is the sustained dense matrix-core rate.  The plain
//    forms use constant operands; the _random forms give every lane and chain
//    its own pseudo-random operands (i8: any code; bf16: random sign and
//    mantissa, magnitudes in [1/4, 4)), which switch the matrix cores as real
//    data does: they draw more power and the part holds a lower clock.
//  * tqp_graph_time: captures a caller's launches into a hipGraph and times its
//    replays with events on the capture stream.
//  * tqp_gemm_w8a8_phases: one launch of the library's W8A8 GEMM kernel
//    (tq_gemm_dma.h, the same source as libtq.so's) instantiated with per-wave
//    real-time stamps: start, first stage landed, end of the K loop, end of the
//    epilogue.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../tq_gemm_dma.h"

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

// The INT4 GEMV's own access pattern with its arithmetic left out: 1024-thread
// blocks, block b owns the 16 * kLoads KB at b * that, wave w of it the kLoads
// consecutive 1 KB pieces at w * kLoads KB (lane l: bytes 16 l .. 16 l + 15 of
// each piece), kWin loads in flight per lane and the next one issued as the
// oldest is consumed; the values are xor-folded, one word per block.  Pieces
// past the end re-read the last one.
template <int kLoads, int kWin>
__global__ __launch_bounds__(1024) void k_hbm_read_waves(const u32x4* __restrict__ p, int64_t n16,
                                                         uint32_t* __restrict__ out) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t base = (static_cast<int64_t>(blockIdx.x) * 16 + wave) * kLoads * 64 + lane;
    auto at = [&](int i) { return p + min<int64_t>(base + i * 64, n16 - 1); };
    u32x4 w[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) w[i] = __builtin_nontemporal_load(at(i));
    u32x4 acc = u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
        acc ^= w[i % kWin];
        if (i + kWin < kLoads) {
            w[i % kWin] = __builtin_nontemporal_load(at(i + kWin));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    uint32_t r = acc.x ^ acc.y ^ acc.z ^ acc.w;
    for (int o = 32; o > 0; o >>= 1) r ^= __shfl_xor(r, o, 64);
    __shared__ uint32_t part[16];
    if (lane == 0) part[wave] = r;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
        for (int v = 0; v < 16; ++v) s ^= part[v];
        out[blockIdx.x] = s;
    }
}

// The headline INT4 GEMV (one token, 64-row tiles of the tiled layout, 16
// waves per tile splitting K by groups, kGPW groups per wave) with its
// arithmetic left out: the same loads in the same order (the wave's x slice,
// its group scales, its weight pieces kWin at a time), the same staging of x
// in LDS with the DPP group sums, and the same block reduction; the nibble
// unpack and the MFMAs are replaced by an xor fold of the weight pieces.
// out[b * 64 + l] = xor of lane l's 16-byte weight pieces of block b (the value
// tqp_hbm_read_waves produces for the same bytes); out[(gridDim.x + b) * 64 +
// l] folds the x sums and scales, which keeps them live.
template <int kGPW, int kWin>
__global__ __launch_bounds__(1024) void k_gemv_w4_skeleton(const uint16_t* __restrict__ x,
                                                           const uint8_t* __restrict__ pt,
                                                           const uint16_t* __restrict__ st, int64_t k,
                                                           uint32_t* __restrict__ out) {
    constexpr int T = 64, kCPW = 4 * kGPW, kItems = kCPW * 8, kIPL = (kItems + 63) / 64;
    __shared__ __attribute__((aligned(16))) uint8_t xs[16][kCPW * 64 + 16];
    __shared__ uint32_t part[16][64], side[16][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t tile = blockIdx.x, C = k >> 5, G = k >> 7;
    const int64_t g0 = static_cast<int64_t>(wave) * kGPW, c0 = 4 * g0;
    const int row0 = 4 * (lane >> 4) + 16 * (lane & 3);  // any 4 rows of the tile
    uint2 xv[kIPL];
#pragma unroll
    for (int q = 0; q < kIPL; ++q) {
        const int it = min(lane + 64 * q, kItems - 1);
        xv[q] = *reinterpret_cast<const uint2*>(x + min<int64_t>(c0 * 32 + 4 * it, k - 4));
    }
    uint2 sc[kGPW];
#pragma unroll
    for (int g = 0; g < kGPW; ++g) sc[g] = *reinterpret_cast<const uint2*>(st + (tile * G + g0 + g) * T + row0);
    const uint8_t* wb = pt + (tile * C * T + lane) * 16;
    u32x4 w[kWin];
#pragma unroll
    for (int i = 0; i < kWin; ++i) w[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + (c0 + i) * T * 16));
    float gs = 0.0f;
#pragma unroll
    for (int q = 0; q < kIPL; ++q) {
        const int it = lane + 64 * q;
        const uint2 v = xv[q];
        const uint2 p = make_uint2(__builtin_amdgcn_update_dpp(0, static_cast<int>(v.x), 0xB1, 0xF, 0xF, false),
                                   __builtin_amdgcn_update_dpp(0, static_cast<int>(v.y), 0xB1, 0xF, 0xF, false));
        const bool odd = it & 1;
        const uint32_t hi = odd ? v.y : p.x, lo = odd ? p.y : v.x;
        if (it < kItems)
            *reinterpret_cast<uint2*>(&xs[wave][(it >> 1) * 16 + (odd ? 8 : 0)]) =
                make_uint2(__builtin_amdgcn_perm(hi, lo, 0x05040100u), __builtin_amdgcn_perm(hi, lo, 0x07060302u));
        float s = __uint_as_float(v.x << 16) + __uint_as_float(v.x & 0xFFFF0000u) + __uint_as_float(v.y << 16) +
                  __uint_as_float(v.y & 0xFFFF0000u);
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) s += __shfl_xor(s, o, 16);
        gs += s;
    }
    u32x4 acc = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < kCPW; ++i) {
        acc ^= w[i % kWin];
        if (i + kWin < kCPW) {
            w[i % kWin] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wb + (c0 + i + kWin) * T * 16));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    uint32_t sf = __float_as_uint(gs);
#pragma unroll
    for (int g = 0; g < kGPW; ++g) sf ^= sc[g].x ^ sc[g].y;
    part[wave][lane] = acc.x ^ acc.y ^ acc.z ^ acc.w;
    side[wave][lane] = sf ^ xs[wave][lane % (kCPW * 64)];
    __syncthreads();
    if (threadIdx.x < 64) {
        uint32_t a = 0, b = 0;
        for (int v = 0; v < 16; ++v) {
            a ^= part[v][threadIdx.x];
            b ^= side[v][threadIdx.x];
        }
        out[blockIdx.x * 64 + threadIdx.x] = a;
        out[(gridDim.x + blockIdx.x) * 64 + threadIdx.x] = b;
    }
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

// Reads `bytes` in the INT4 GEMV's pattern (k_hbm_read_waves): `loads` 1 KB
// pieces per wave (8 or 16), `window` loads in flight (3 or 8); `out` needs one
// word per block (bytes / (16 KB * loads), rounded up).
int tqp_hbm_read_waves(const void* buf, int64_t bytes, uint32_t* out, int loads, int window, hipStream_t stream) {
    const int64_t n16 = bytes / 16;
    const int64_t per = 1024LL * loads;
    const unsigned blocks = static_cast<unsigned>((n16 + per - 1) / per);
    const u32x4* p = static_cast<const u32x4*>(buf);
    if (loads == 8 && window == 3) k_hbm_read_waves<8, 3><<<blocks, 1024, 0, stream>>>(p, n16, out);
    else if (loads == 8) k_hbm_read_waves<8, 8><<<blocks, 1024, 0, stream>>>(p, n16, out);
    else if (window == 3) k_hbm_read_waves<16, 3><<<blocks, 1024, 0, stream>>>(p, n16, out);
    else k_hbm_read_waves<16, 8><<<blocks, 1024, 0, stream>>>(p, n16, out);
    return static_cast<int>(hipGetLastError());
}

// The headline GEMV's loads without its arithmetic (k_gemv_w4_skeleton): x
// bf16 [k], the tiled weight of n rows (n % 64 == 0, 64-row tiles) and its
// scales, k in {2048, 4096, 8192}; `out` needs 2 * (n / 64) * 64 words.
int tqp_gemv_w4_skeleton(const uint16_t* x, const uint8_t* pt, const uint16_t* st, int64_t n, int64_t k,
                         uint32_t* out, hipStream_t stream) {
    if (n <= 0 || n % 64 != 0 || (k != 2048 && k != 4096 && k != 8192)) return static_cast<int>(hipErrorInvalidValue);
    const unsigned tiles = static_cast<unsigned>(n / 64);
    if (k == 2048) k_gemv_w4_skeleton<1, 3><<<tiles, 1024, 0, stream>>>(x, pt, st, k, out);
    else if (k == 4096) k_gemv_w4_skeleton<2, 3><<<tiles, 1024, 0, stream>>>(x, pt, st, k, out);
    else k_gemv_w4_skeleton<4, 3><<<tiles, 1024, 0, stream>>>(x, pt, st, k, out);
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

// One launch of k_gemm_w8a8_dma<true> at M x N x K (M % 128 == 0, N % 256 == 0,
// K % 128 == 0; the library's dispatch runs this kernel at those shapes): qa [M,
// K] and qw [N, K] int8 codes, sa [M] and sw [N] scales, y f32 [M, N]; ts
// receives 6 words per wave, (M / 128) (N / 256) 4 waves: the real-time clock
// (100 MHz) at the wave's start, once the first stage has landed, after the K
// loop and after the epilogue's stores, then the wave's HW_ID register and 0.
int tqp_gemm_w8a8_phases(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw, int m, int n, int k,
                         float* y, uint64_t* ts, hipStream_t stream) {
    if (m <= 0 || n <= 0 || k <= 0 || m % 128 != 0 || n % 256 != 0 || k % 128 != 0 || !ts)
        return static_cast<int>(hipErrorInvalidValue);
    const int tm = m / 128, tn = n / 256;
    tq::k_gemm_w8a8_dma<true><<<tm * tn, 256, 0, stream>>>(qa, sa, qw, sw, nullptr, m, n, k, nullptr, y, tm, tn,
                                                           ts);
    return static_cast<int>(hipGetLastError());
}

// Graph timing without a framework in between: `launch(i, stream)` enqueues
// step i on `stream` (it may call any library entry point).  Runs `warmup`
// steps eagerly, captures `steps` steps into one hipGraph, replays it once, then
// times `reps` replays with events recorded on the same stream and writes each
// replay's microseconds per step to us[0 .. reps).  The stream is created here
// at the default priority and destroyed before returning.  Returns a hipError_t
// (hipErrorUnknown when `launch` reports a nonzero status).
typedef int (*tqp_launch_fn)(int step, void* stream);

int tqp_graph_time(tqp_launch_fn launch, int steps, int warmup, int reps, float* us) {
    if (!launch || steps <= 0 || reps <= 0 || !us) return static_cast<int>(hipErrorInvalidValue);
    hipStream_t s = nullptr;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t err = hipStreamCreate(&s);
    auto run = [&](int i) { return launch(i, s) == 0 ? hipSuccess : hipErrorUnknown; };
    for (int i = 0; i < warmup && err == hipSuccess; ++i) err = run(i);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err == hipSuccess) err = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
    if (err == hipSuccess) {
        hipError_t cap = hipSuccess;
        for (int i = 0; i < steps && cap == hipSuccess; ++i) cap = run(i);
        err = hipStreamEndCapture(s, &g);  // ends the capture whatever the launches reported
        if (err == hipSuccess) err = cap;
    }
    if (err == hipSuccess) err = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (err == hipSuccess) err = hipGraphLaunch(ge, s);
    if (err == hipSuccess) err = hipStreamSynchronize(s);
    if (err == hipSuccess) err = hipEventCreate(&e0);
    if (err == hipSuccess) err = hipEventCreate(&e1);
    for (int r = 0; r < reps && err == hipSuccess; ++r) {
        err = hipEventRecord(e0, s);
        if (err == hipSuccess) err = hipGraphLaunch(ge, s);
        if (err == hipSuccess) err = hipEventRecord(e1, s);
        if (err == hipSuccess) err = hipEventSynchronize(e1);
        float ms = 0.0f;
        if (err == hipSuccess) err = hipEventElapsedTime(&ms, e0, e1);
        us[r] = ms * 1000.0f / static_cast<float>(steps);
    }
    if (s) hipStreamSynchronize(s);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (ge) hipGraphExecDestroy(ge);
    if (g) hipGraphDestroy(g);
    if (s) hipStreamDestroy(s);
    return static_cast<int>(err);
}

}  // extern "C"
