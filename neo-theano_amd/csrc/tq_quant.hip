// tq_quant.hip -- quantize / dequantize kernels for gfx950 and their C ABI.
//
// Reference semantics: crates/theano-quantize/src/quantize.rs:8-55 and
// observer.rs:42-136 (f64, round half away from zero, clamp).  The hot
// formats (per-row INT8, INT4 group-128) use an exact f32 rounding (rhaz_div)
// instead of f64 division; the generic primitives compute in f64 directly.
//
// All kernels are HBM-bound streams: each lane moves 16-byte vectors, rows or
// groups are reduced with wave64 butterflies, and codes are packed in
// registers before one coalesced store.
#include <cmath>

#include "tq_internal.h"
#include "tq_rowfmt.h"

#pragma clang fp contract(off)

namespace tq {
namespace {

constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

// Block-wide max of a per-thread value (NaN-free inputs), result in every thread.
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kWavesPerBlock; ++i) r = fmaxf(r, red[i]);
    return r;
}

// ---- per-row quantize, register-cached row (K % 4 == 0, K <= 1024 * kItems) ----
// 256-thread blocks, block b taking rows b, b + gridDim.x, ... (one row per
// block when the grid has a block per row); each thread holds kItems f32x4 of
// the row.  A block requests its next row once the current one is coded and
// stored (codes only, 4096 x 4096: 15.4-16.0 us with 2048 blocks of two rows
// each, against 16.7 us for one block per row and 15.9 us with the next row's
// loads issued before the current row's reduction).  The
// block reduction alternates between two LDS slots, so a wave that runs ahead
// into the next row never overwrites a maximum another wave has still to read.
// Serves K other than 2048 and 4096, which take k_quant_rows_split.
template <class Fmt, int kItems>
__global__ __launch_bounds__(kBlock) void k_quant_rows_vec(const float* __restrict__ w, int64_t rows, int64_t k,
                                                           typename Fmt::code_t* __restrict__ q,
                                                           float* __restrict__ s, float* __restrict__ w_hat) {
    __shared__ float red[2][kWavesPerBlock];
    const int k4 = static_cast<int>(k >> 2);
    int par = 0;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x, par ^= 1) {
        const f32x4* src = reinterpret_cast<const f32x4*>(w + row * k);
        f32x4 v[kItems];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int idx = threadIdx.x + i * kBlock;
            if (idx < k4) {
                v[i] = __builtin_nontemporal_load(src + idx);
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
            }
        }
        const float sc = row_scale<Fmt>(absmax_finish(block_max(m, red[par])));
        if (threadIdx.x == 0) s[row] = sc;
        const typename Fmt::Row coder(sc);
        uint32_t* qd = reinterpret_cast<uint32_t*>(q + row * k);
        f32x4* wd = reinterpret_cast<f32x4*>(w_hat + row * k);
#pragma unroll
        for (int i = 0; i < kItems; ++i) {
            const int idx = threadIdx.x + i * kBlock;
            if (idx < k4) {
                const uint32_t c = coder.code4(v[i]);
                if (q) __builtin_nontemporal_store(c, qd + idx);
                if (w_hat) __builtin_nontemporal_store(Fmt::value4(c, sc), wd + idx);
            }
        }
    }
}

// ---- per-row quantize, one wave per row (codes only, K % 4 == 0, K <= 256 kI) ----
// 128-thread blocks of two waves; wave w takes rows w, w + (waves in the grid),
// ...; lane l holds f32x4 items l + 64 i of the row, so every wave-wide load
// reads 1 KB contiguously, and the row maximum is a wave reduction (no LDS, no
// barrier).  Serves K that is not 2048 or 4096 (those take k_quant_rows_split).
template <class Fmt, int kI>
__global__ __launch_bounds__(128) void k_quant_rows_wave(const float* __restrict__ w, int64_t rows, int64_t k,
                                                         typename Fmt::code_t* __restrict__ q,
                                                         float* __restrict__ s) {
    const int lane = threadIdx.x & 63;
    const int k4 = static_cast<int>(k >> 2);
    const int64_t nw = static_cast<int64_t>(gridDim.x) * 2;
    for (int64_t row = static_cast<int64_t>(blockIdx.x) * 2 + (threadIdx.x >> 6); row < rows; row += nw) {
        const f32x4* src = reinterpret_cast<const f32x4*>(w + row * k);
        // every load is issued (lanes past the row re-read its last item, which
        // leaves the maximum unchanged): a load under a lane mask made the compiler
        // wait for each one before the next (14.4 against 10.1 us at 2048 x 4096)
        f32x4 v[kI];
        float m = -INFINITY;
#pragma unroll
        for (int i = 0; i < kI; ++i)
            v[i] = __builtin_nontemporal_load(src + min(lane + 64 * i, k4 - 1));
#pragma unroll
        for (int i = 0; i < kI; ++i)
            m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        const float sc = row_scale<Fmt>(absmax_finish(wave_max(m)));
        if (lane == 0) s[row] = sc;
        const typename Fmt::Row coder(sc);
        uint32_t* qd = reinterpret_cast<uint32_t*>(q + row * k);
#pragma unroll
        for (int i = 0; i < kI; ++i) {
            const int idx = lane + 64 * i;
            if (idx < k4) __builtin_nontemporal_store(coder.code4(v[i]), qd + idx);
        }
    }
}

// ---- per-row quantize, one row per block of kW waves (K == 256 kI kW) ----
// Wave v holds the v-th kW-th of the row (lane l: f32x4 items l + 64 i of it);
// the wave maxima meet in LDS; codes, and the dequantized copy when w_hat is
// given.  A row's coding starts only once its last bytes are in, so the launch
// ends with the coding of the rows that land last: spread over kW waves, that
// tail is 1/kW of a wave-per-row kernel's.  At 2048 x 4096 (the W8A8
// activations): 8.7-8.8 us with 4 waves per row, 8.8-8.9 with 2, 9.4-9.5 with 8
// and 9.2 with a wave per row; the same loads and stores with the coder
// replaced by a trivial fold take 8.1 us, a plain read of the 42 MB 8.0 us.
template <class Fmt, int kI, int kW>
__global__ __launch_bounds__(64 * kW) void k_quant_rows_split(const float* __restrict__ w, int64_t k,
                                                              typename Fmt::code_t* __restrict__ q,
                                                              float* __restrict__ s, float* __restrict__ w_hat) {
    __shared__ float red[kW];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t row = blockIdx.x;
    const f32x4* src = reinterpret_cast<const f32x4*>(w + row * k) + wave * 64 * kI;
    f32x4 v[kI];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kI; ++i) v[i] = __builtin_nontemporal_load(src + lane + 64 * i);
#pragma unroll
    for (int i = 0; i < kI; ++i)
        m = fmaxf(m, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int j = 1; j < kW; ++j) m = fmaxf(m, red[j]);
    const float sc = row_scale<Fmt>(absmax_finish(m));
    if (threadIdx.x == 0) s[row] = sc;
    const typename Fmt::Row coder(sc);
    uint32_t* qd = reinterpret_cast<uint32_t*>(q + row * k) + wave * 64 * kI;
#pragma unroll
    for (int i = 0; i < kI; ++i) {
        const uint32_t c = coder.code4(v[i]);
        __builtin_nontemporal_store(c, qd + lane + 64 * i);
        if (w_hat)
            __builtin_nontemporal_store(Fmt::value4(c, sc),
                                        reinterpret_cast<f32x4*>(w_hat + row * k) + wave * 64 * kI + lane + 64 * i);
    }
}

// ---- per-row quantize, any K / alignment: two passes over the row ----
template <class Fmt>
__global__ __launch_bounds__(kBlock) void k_quant_rows_generic(const float* __restrict__ w, int64_t k,
                                                               typename Fmt::code_t* __restrict__ q,
                                                               float* __restrict__ s, float* __restrict__ w_hat) {
    __shared__ float red[kWavesPerBlock];
    const int64_t row = blockIdx.x;
    const float* src = w + row * k;
    float m = -INFINITY;
    for (int64_t i = threadIdx.x; i < k; i += kBlock) m = fmaxf(m, fabsf(src[i]));
    const float sc = row_scale<Fmt>(absmax_finish(block_max(m, red)));
    if (threadIdx.x == 0) s[row] = sc;
    const typename Fmt::Row coder(sc);
    for (int64_t i = threadIdx.x; i < k; i += kBlock) {
        const typename Fmt::code_t c = coder.code1(src[i]);
        if (q) q[row * k + i] = c;
        if (w_hat) w_hat[row * k + i] = Fmt::value1(c, sc);
    }
}

// ---- per-row dequant: w_hat = f32(value(q) * s[row]) ----
// Vector form: 16 codes per thread (K % 16 == 0, aligned).
// Thread t of a block handles 4-element units t + 256 j (j < kDqUnits): every
// wave-wide load reads 256 contiguous code bytes, every store writes 1 KB.
constexpr int kDqUnits = 4;
template <class Fmt>
__global__ __launch_bounds__(kBlock) void k_dequant_rows_vec(const typename Fmt::code_t* __restrict__ q,
                                                             const float* __restrict__ s, int64_t k, int64_t n4,
                                                             float* __restrict__ w_hat) {
    const int64_t u0 = static_cast<int64_t>(blockIdx.x) * (kBlock * kDqUnits) + threadIdx.x;
    uint32_t c[kDqUnits];
    float sc[kDqUnits];
#pragma unroll
    for (int j = 0; j < kDqUnits; ++j) {
        const int64_t u = min<int64_t>(u0 + j * kBlock, n4 - 1);
        c[j] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(q) + u);
        sc[j] = s[(u * 4) / k];
    }
#pragma unroll
    for (int j = 0; j < kDqUnits; ++j) {
        const int64_t u = u0 + j * kBlock;
        if (u >= n4) break;
        __builtin_nontemporal_store(Fmt::value4(c[j], sc[j]), reinterpret_cast<f32x4*>(w_hat) + u);
    }
}

template <class Fmt>
__global__ __launch_bounds__(kBlock) void k_dequant_rows_generic(const typename Fmt::code_t* __restrict__ q,
                                                                 const float* __restrict__ s, int64_t k,
                                                                 int64_t total, float* __restrict__ w_hat) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= total) return;
    w_hat[i] = Fmt::value1(q[i], s[i / k]);
}

// ---- INT4 group-128: 16 lanes per group, 8 consecutive elements per lane ----
__device__ __forceinline__ uint16_t scale_i4_bits(float absmax) {
    const float sf = static_cast<float>(static_cast<double>(absmax) / 7.0);
    uint16_t h = __half_as_ushort(__float2half_rn(sf));
    return h == 0 ? uint16_t(1) : h;  // floor at 2^-24, the smallest positive f16
}

__global__ __launch_bounds__(kBlock) void k_quant_i4_g128(const float* __restrict__ w,
                                                          int64_t groups,
                                                          uint8_t* __restrict__ packed,
                                                          uint16_t* __restrict__ s16,
                                                          float* __restrict__ w_hat) {
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const int64_t g = slot >> 4;
    const bool valid = g < groups;
    float x[8];
    float m = -INFINITY;
    if (valid) {
        const f32x4* p = reinterpret_cast<const f32x4*>(w) + slot * 2;
        const f32x4 a = __builtin_nontemporal_load(p);
        const f32x4 b = __builtin_nontemporal_load(p + 1);
        x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
#pragma unroll
        for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(x[i]));
    }
    m = group_max<16>(m);  // all 16 lanes of a group are valid or invalid together
    if (!valid) return;
    const uint16_t hb = scale_i4_bits(absmax_finish(m));
    const float sc = __half2float(__ushort_as_half(hb));
    if ((threadIdx.x & 15) == 0) s16[g] = hb;
    int c[8];
    if (sc < INFINITY) {
        const float inv = 1.0f / sc, half = 0.5f * sc;
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = signed_code(x[i], rhaz_div(fabsf(x[i]), sc, inv, half, 32.0f), -8, 7);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) c[i] = 0;
    }
    if (packed) {
        uint32_t word = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) word |= static_cast<uint32_t>(c[i] & 0xF) << (4 * i);
        reinterpret_cast<uint32_t*>(packed)[slot] = word;
    }
    if (w_hat) {
        f32x4* d = reinterpret_cast<f32x4*>(w_hat) + slot * 2;
        d[0] = f32x4{c[0] * sc, c[1] * sc, c[2] * sc, c[3] * sc};
        d[1] = f32x4{c[4] * sc, c[5] * sc, c[6] * sc, c[7] * sc};
    }
}

// 8 codes (one packed dword) per thread.
__global__ __launch_bounds__(kBlock) void k_dequant_i4_g128(const uint8_t* __restrict__ packed,
                                                            const uint16_t* __restrict__ s16,
                                                            int64_t slots,
                                                            float* __restrict__ w_hat) {
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (slot >= slots) return;
    const float sc = __half2float(__ushort_as_half(s16[slot >> 4]));
    const uint32_t word = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(packed) + slot);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int nib = static_cast<int>((word >> (4 * i)) & 0xF);
        o[i] = static_cast<float>(nib >= 8 ? nib - 16 : nib) * sc;
    }
    f32x4* d = reinterpret_cast<f32x4*>(w_hat) + slot * 2;
    d[0] = f32x4{o[0], o[1], o[2], o[3]};
    d[1] = f32x4{o[4], o[5], o[6], o[7]};
}

// ---- generic reference primitives, f64 arithmetic ----
// Rust f64::clamp: keeps NaN (comparisons with NaN are false).
__device__ __forceinline__ double rust_clamp(double v, double lo, double hi) {
    v = (v < lo) ? lo : v;
    v = (v > hi) ? hi : v;
    return v;
}

// ---- generic primitives: f64 arithmetic, elements f32 or f64 (TI in, TO out) ----

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void k_quantize_tensor(const TI* __restrict__ x, int64_t n, double scale,
                                                            double zp, double qmin, double qmax,
                                                            TO* __restrict__ q) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        q[i] = static_cast<TO>(rust_clamp(round(static_cast<double>(x[i]) / scale + zp), qmin, qmax));
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void k_dequantize_tensor(const TI* __restrict__ q, int64_t n, double scale,
                                                              double zp, TO* __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        out[i] = static_cast<TO>((static_cast<double>(q[i]) - zp) * scale);
}

template <typename TI, typename TO>
__global__ __launch_bounds__(kBlock) void k_fake_quantize(const TI* __restrict__ x, int64_t n, double scale,
                                                          double zp, double qmin, double qmax,
                                                          TO* __restrict__ out) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const double c = rust_clamp(round(static_cast<double>(x[i]) / scale + zp), qmin, qmax);
        out[i] = static_cast<TO>((c - zp) * scale);
    }
}

// NaN-ignoring min / max (f64::min / f64::max, fminf / fmin)
__device__ __forceinline__ float vmin(float a, float b) { return fminf(a, b); }
__device__ __forceinline__ float vmax(float a, float b) { return fmaxf(a, b); }
__device__ __forceinline__ double vmin(double a, double b) { return fmin(a, b); }
__device__ __forceinline__ double vmax(double a, double b) { return fmax(a, b); }

// Block-wide NaN-ignoring min and max, results valid in thread 0.
template <typename T>
__device__ __forceinline__ void block_minmax(T& mn, T& mx, T* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        mn = vmin(mn, __shfl_xor(mn, o, kWave));
        mx = vmax(mx, __shfl_xor(mx, o, kWave));
    }
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) {
        red[2 * wid] = mn;
        red[2 * wid + 1] = mx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int i = 1; i < kWavesPerBlock; ++i) {
            mn = vmin(mn, red[2 * i]);
            mx = vmax(mx, red[2 * i + 1]);
        }
    }
}

// Order-preserving integer keys of non-NaN values (atomic min/max on integers).
template <typename T>
struct OrderedKey;
template <>
struct OrderedKey<float> {
    using K = int;
    __device__ static K key(float f) {
        const int b = __float_as_int(f);
        return b >= 0 ? b : b ^ 0x7FFFFFFF;
    }
    __device__ static float val(K k) { return __int_as_float(k >= 0 ? k : k ^ 0x7FFFFFFF); }
};
template <>
struct OrderedKey<double> {
    using K = long long;
    __device__ static K key(double f) {
        const long long b = __double_as_longlong(f);
        return b >= 0 ? b : b ^ 0x7FFFFFFFFFFFFFFFLL;
    }
    __device__ static double val(K k) { return __longlong_as_double(k >= 0 ? k : k ^ 0x7FFFFFFFFFFFFFFFLL); }
};

// workspace layout for quantize_per_tensor: keys {min, max}
template <typename T>
__global__ void k_per_tensor_init(typename OrderedKey<T>::K* ws) {
    if (threadIdx.x == 0) {
        ws[0] = OrderedKey<T>::key(static_cast<T>(INFINITY));
        ws[1] = OrderedKey<T>::key(static_cast<T>(-INFINITY));
    }
}

// NaN-ignoring min/max of x folded into keys (one atomic pair per block).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_minmax_keys(const T* __restrict__ x, int64_t n,
                                                        typename OrderedKey<T>::K* ws) {
    __shared__ T red[2 * kWavesPerBlock];
    T mn = static_cast<T>(INFINITY), mx = static_cast<T>(-INFINITY);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const T v = x[i];
        mn = vmin(mn, v);
        mx = vmax(mx, v);
    }
    block_minmax(mn, mx, red);
    if (threadIdx.x == 0) {
        atomicMin(ws, OrderedKey<T>::key(mn));
        atomicMax(ws + 1, OrderedKey<T>::key(mx));
    }
}

// quantize.rs:33-40: scale = max((max-min)/(qmax-qmin), 1e-10), zp = clamp(round(qmin - min/scale))
template <typename T>
__device__ __forceinline__ void per_tensor_params(const typename OrderedKey<T>::K* ws, double qmin, double qmax,
                                                  double* scale, double* zp) {
    const double mn = static_cast<double>(OrderedKey<T>::val(ws[0]));
    const double mx = static_cast<double>(OrderedKey<T>::val(ws[1]));
    const double s = fmax((mx - mn) / (qmax - qmin), 1e-10);
    *scale = s;
    *zp = rust_clamp(round(qmin - mn / s), qmin, qmax);
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_per_tensor_quantize(const T* __restrict__ x, int64_t n,
                                                                const typename OrderedKey<T>::K* ws,
                                                                double qmin, double qmax, T* __restrict__ q,
                                                                double* scale_zp) {
    double s, zp;
    per_tensor_params<T>(ws, qmin, qmax, &s, &zp);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
        scale_zp[0] = s;
        scale_zp[1] = zp;
    }
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride)
        q[i] = static_cast<T>(rust_clamp(round(static_cast<double>(x[i]) / s + zp), qmin, qmax));
}

// ---- observers: state = channels x {min, max} ----
template <typename T>
__global__ void k_minmax_reset(T* state, int64_t channels) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (c < channels) {
        state[2 * c] = static_cast<T>(INFINITY);
        state[2 * c + 1] = static_cast<T>(-INFINITY);
    }
}

// Folds a block's min/max into state[0..1] with compare-and-swap loops.
__device__ __forceinline__ unsigned int as_bits(float v) { return __float_as_uint(v); }
__device__ __forceinline__ unsigned long long as_bits(double v) {
    return static_cast<unsigned long long>(__double_as_longlong(v));
}
__device__ __forceinline__ float from_bits(unsigned int b, float) { return __uint_as_float(b); }
__device__ __forceinline__ double from_bits(unsigned long long b, double) {
    return __longlong_as_double(static_cast<long long>(b));
}

template <bool kMax, typename T>
__device__ void atomic_fold(T* addr, T v) {
    using U = decltype(as_bits(v));
    U* a = reinterpret_cast<U*>(addr);
    U old = __atomic_load_n(a, __ATOMIC_RELAXED);
    while (kMax ? (v > from_bits(old, v)) : (v < from_bits(old, v))) {
        const U prev = atomicCAS(a, old, as_bits(v));
        if (prev == old) break;
        old = prev;
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_minmax_observe(const T* __restrict__ x, int64_t n, T* state) {
    __shared__ T red[2 * kWavesPerBlock];
    T mn = static_cast<T>(INFINITY), mx = static_cast<T>(-INFINITY);
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += stride) {
        const T v = x[i];
        mn = vmin(mn, v);
        mx = vmax(mx, v);
    }
    block_minmax(mn, mx, red);
    if (threadIdx.x == 0) {
        atomic_fold<false>(state, mn);
        atomic_fold<true>(state + 1, mx);
    }
}

// One block per channel; channel c covers x[c*per, (c+1)*per).
template <typename T>
__global__ __launch_bounds__(kBlock) void k_minmax_observe_per_channel(const T* __restrict__ x, int64_t per,
                                                                       T* state) {
    __shared__ T red[2 * kWavesPerBlock];
    const int64_t c = blockIdx.x;
    const T* src = x + c * per;
    T mn = static_cast<T>(INFINITY), mx = static_cast<T>(-INFINITY);
    for (int64_t i = threadIdx.x; i < per; i += kBlock) {
        const T v = src[i];
        mn = vmin(mn, v);
        mx = vmax(mx, v);
    }
    block_minmax(mn, mx, red);
    if (threadIdx.x == 0) {
        state[2 * c] = vmin(state[2 * c], mn);
        state[2 * c + 1] = vmax(state[2 * c + 1], mx);
    }
}

int grid_for(int64_t n, int64_t per_block, int64_t cap) {
    int64_t g = (n + per_block - 1) / per_block;
    if (g > cap) g = cap;
    return static_cast<int>(g < 1 ? 1 : g);
}

int qrange(int qdtype, double* qmin, double* qmax) {
    return tq_qdtype_info(qdtype, nullptr, nullptr, qmin, qmax);
}

template <class Fmt>
int launch_quant_rows(const float* w, int64_t rows, int64_t k, typename Fmt::code_t* q, float* s, float* w_hat,
                      hipStream_t st, const char* what) {
    TQ_REQUIRE(rows >= 0 && k >= 0, "%s: negative shape [%lld, %lld]", what, (long long)rows,
               (long long)k);
    TQ_REQUIRE(rows < (int64_t(1) << 31), "%s: too many rows (%lld)", what, (long long)rows);
    if (rows == 0) return TQ_OK;
    TQ_REQUIRE(w && s, "%s: null pointer", what);
    const bool vec = (k % 16 == 0) && k > 0 && k <= 16384 && aligned(w, 16) &&
                     (!q || aligned(q, 4)) && (!w_hat || aligned(w_hat, 16));
    const dim3 grid(static_cast<unsigned>(rows)), block(kBlock);
    const int64_t cus = device_cu_count();
    if (vec && q && (k == 2048 || k == 4096)) {
        // a row per 4-wave block, with or without the dequantized copy: W8A8
        // activations 2048 x 4096 8.8 us; 4096 x 4096 codes 15.7 us and round trip
        // 26.1 us, against 16.3 / 26.8 us for the persistent and per-row blocks below
        constexpr int kSplitW = 4;
        if (k == 2048)
            k_quant_rows_split<Fmt, 8 / kSplitW, kSplitW><<<grid, 64 * kSplitW, 0, st>>>(w, k, q, s, w_hat);
        else
            k_quant_rows_split<Fmt, 16 / kSplitW, kSplitW><<<grid, 64 * kSplitW, 0, st>>>(w, k, q, s, w_hat);
    } else if (vec && !w_hat && k > 1024 && k <= 4096 && rows <= 8 * cus) {
        // codes only, other K of 1-4 K elements, at most 8 rows per CU: a wave per
        // row.  Past that the persistent blocks below stay ahead (4096 x 4096: 17.3
        // us, against 17.9 with two rows per wave and 20.3 with one, 64 MB in flight
        // at once).
        const unsigned g = static_cast<unsigned>((rows + 1) / 2);
        if (k < 2048)
            k_quant_rows_wave<Fmt, 8><<<g, 128, 0, st>>>(w, rows, k, q, s);
        else
            k_quant_rows_wave<Fmt, 16><<<g, 128, 0, st>>>(w, rows, k, q, s);
    } else if (vec) {
        const int64_t items = (k / 4 + kBlock - 1) / kBlock;
        // codes only: persistent, at most 8 blocks per CU, each taking every
        // gridDim-th row; with the dequantized copy as well (twice the stores) one
        // block per row measured faster (25.9 against 26.5 us at 4096 x 4096)
        const int64_t nb = w_hat ? rows : std::min<int64_t>(rows, 8 * cus);
        const dim3 pgrid(static_cast<unsigned>(nb));
        if (items <= 1) k_quant_rows_vec<Fmt, 1><<<pgrid, block, 0, st>>>(w, rows, k, q, s, w_hat);
        else if (items <= 2) k_quant_rows_vec<Fmt, 2><<<pgrid, block, 0, st>>>(w, rows, k, q, s, w_hat);
        else if (items <= 4) k_quant_rows_vec<Fmt, 4><<<pgrid, block, 0, st>>>(w, rows, k, q, s, w_hat);
        else if (items <= 8) k_quant_rows_vec<Fmt, 8><<<pgrid, block, 0, st>>>(w, rows, k, q, s, w_hat);
        else k_quant_rows_vec<Fmt, 16><<<pgrid, block, 0, st>>>(w, rows, k, q, s, w_hat);
    } else {
        k_quant_rows_generic<Fmt><<<grid, block, 0, st>>>(w, k, q, s, w_hat);
    }
    return check_launch(what);
}

template <class Fmt>
int launch_dequant_rows(const typename Fmt::code_t* q, const float* s, int64_t rows, int64_t k, float* w_hat,
                        hipStream_t st, const char* what) {
    TQ_REQUIRE(rows >= 0 && k >= 0, "%s: negative shape", what);
    const int64_t total = rows * k;
    if (total == 0) return TQ_OK;
    TQ_REQUIRE(q && s && w_hat, "%s: null pointer", what);
    if (k % 16 == 0 && aligned(q, 16) && aligned(w_hat, 16)) {
        const int64_t n4 = total / 4;
        k_dequant_rows_vec<Fmt><<<grid_for(n4, kBlock * kDqUnits, INT32_MAX), kBlock, 0, st>>>(q, s, k, n4, w_hat);
    } else {
        k_dequant_rows_generic<Fmt><<<grid_for(total, kBlock, INT32_MAX), kBlock, 0, st>>>(q, s, k, total, w_hat);
    }
    return check_launch(what);
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" {

int tq_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q, float* s,
                           tq_stream_t stream) {
    if (rows > 0 && k > 0 && !q) return fail(TQ_EINVAL, "tq_quantize_i8_rowwise: null q");
    return launch_quant_rows<FmtI8>(w, rows, k, q, s, nullptr, as_hip(stream), "tq_quantize_i8_rowwise");
}

int tq_fake_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q, float* s,
                                float* w_hat, tq_stream_t stream) {
    if (rows > 0 && k > 0 && (!q || !w_hat))
        return fail(TQ_EINVAL, "tq_fake_quantize_i8_rowwise: null output");
    return launch_quant_rows<FmtI8>(w, rows, k, q, s, w_hat, as_hip(stream), "tq_fake_quantize_i8_rowwise");
}

int tq_dequantize_i8_rowwise(const int8_t* q, const float* s, int64_t rows, int64_t k,
                             float* w_hat, tq_stream_t stream) {
    return launch_dequant_rows<FmtI8>(q, s, rows, k, w_hat, as_hip(stream), "tq_dequantize_i8_rowwise");
}

int tq_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q, float* s,
                            tq_stream_t stream) {
    if (rows > 0 && k > 0 && !q) return fail(TQ_EINVAL, "tq_quantize_fp8_rowwise: null q");
    return launch_quant_rows<FmtFp8>(w, rows, k, q, s, nullptr, as_hip(stream), "tq_quantize_fp8_rowwise");
}

int tq_fake_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q, float* s,
                                 float* w_hat, tq_stream_t stream) {
    if (rows > 0 && k > 0 && (!q || !w_hat))
        return fail(TQ_EINVAL, "tq_fake_quantize_fp8_rowwise: null output");
    return launch_quant_rows<FmtFp8>(w, rows, k, q, s, w_hat, as_hip(stream), "tq_fake_quantize_fp8_rowwise");
}

int tq_dequantize_fp8_rowwise(const uint8_t* q, const float* s, int64_t rows, int64_t k,
                              float* w_hat, tq_stream_t stream) {
    return launch_dequant_rows<FmtFp8>(q, s, rows, k, w_hat, as_hip(stream), "tq_dequantize_fp8_rowwise");
}

int tq_quantize_i4_g128(const float* w, int64_t rows, int64_t k, uint8_t* packed,
                        uint16_t* s_f16, tq_stream_t stream) {
    TQ_REQUIRE(rows >= 0 && k >= 0, "tq_quantize_i4_g128: negative shape");
    TQ_REQUIRE(k % 128 == 0, "tq_quantize_i4_g128: K=%lld is not a multiple of the group size 128",
               (long long)k);
    const int64_t groups = rows * (k / 128);
    if (groups == 0) return TQ_OK;
    TQ_REQUIRE(w && packed && s_f16, "tq_quantize_i4_g128: null pointer");
    TQ_REQUIRE(aligned(w, 16) && aligned(packed, 4) && aligned(s_f16, 2),
               "tq_quantize_i4_g128: misaligned pointer (W 16 B, packed 4 B, scales 2 B)");
    k_quant_i4_g128<<<grid_for(groups * 16, kBlock, INT32_MAX), kBlock, 0, as_hip(stream)>>>(
        w, groups, packed, s_f16, nullptr);
    return check_launch("tq_quantize_i4_g128");
}

int tq_dequantize_i4_g128(const uint8_t* packed, const uint16_t* s_f16, int64_t rows, int64_t k,
                          float* w_hat, tq_stream_t stream) {
    TQ_REQUIRE(rows >= 0 && k >= 0, "tq_dequantize_i4_g128: negative shape");
    TQ_REQUIRE(k % 128 == 0, "tq_dequantize_i4_g128: K=%lld is not a multiple of 128", (long long)k);
    const int64_t slots = rows * (k / 8);
    if (slots == 0) return TQ_OK;
    TQ_REQUIRE(packed && s_f16 && w_hat, "tq_dequantize_i4_g128: null pointer");
    TQ_REQUIRE(aligned(packed, 4) && aligned(w_hat, 16) && aligned(s_f16, 2),
               "tq_dequantize_i4_g128: misaligned pointer (packed 4 B, W_hat 16 B)");
    k_dequant_i4_g128<<<grid_for(slots, kBlock, INT32_MAX), kBlock, 0, as_hip(stream)>>>(
        packed, s_f16, slots, w_hat);
    return check_launch("tq_dequantize_i4_g128");
}

}  // extern "C"

namespace tq {
namespace {

template <typename TI, typename TO>
int quantize_tensor_impl(const TI* x, int64_t n, double scale, double zero_point, int qdtype, TO* q,
                         tq_stream_t stream, const char* what) {
    double qmin, qmax;
    const int st = qrange(qdtype, &qmin, &qmax);
    if (st != TQ_OK) return st;
    TQ_REQUIRE(n >= 0, "%s: negative size", what);
    if (n == 0) return TQ_OK;
    TQ_REQUIRE(x && q, "%s: null pointer", what);
    k_quantize_tensor<TI, TO><<<grid_for(n, kBlock, 65536), kBlock, 0, as_hip(stream)>>>(x, n, scale, zero_point,
                                                                                         qmin, qmax, q);
    return check_launch(what);
}

template <typename TI, typename TO>
int dequantize_tensor_impl(const TI* q, int64_t n, double scale, double zero_point, TO* out, tq_stream_t stream,
                           const char* what) {
    TQ_REQUIRE(n >= 0, "%s: negative size", what);
    if (n == 0) return TQ_OK;
    TQ_REQUIRE(q && out, "%s: null pointer", what);
    k_dequantize_tensor<TI, TO><<<grid_for(n, kBlock, 65536), kBlock, 0, as_hip(stream)>>>(q, n, scale,
                                                                                           zero_point, out);
    return check_launch(what);
}

template <typename TI, typename TO>
int fake_quantize_impl(const TI* x, int64_t n, double scale, double zero_point, int qdtype, TO* out,
                       tq_stream_t stream, const char* what) {
    double qmin, qmax;
    const int st = qrange(qdtype, &qmin, &qmax);
    if (st != TQ_OK) return st;
    TQ_REQUIRE(n >= 0, "%s: negative size", what);
    if (n == 0) return TQ_OK;
    TQ_REQUIRE(x && out, "%s: null pointer", what);
    k_fake_quantize<TI, TO><<<grid_for(n, kBlock, 65536), kBlock, 0, as_hip(stream)>>>(x, n, scale, zero_point,
                                                                                       qmin, qmax, out);
    return check_launch(what);
}

template <typename T>
int quantize_per_tensor_impl(const T* x, int64_t n, int qdtype, T* q, double* scale_zp, void* workspace,
                             tq_stream_t stream, const char* what) {
    double qmin, qmax;
    const int st = qrange(qdtype, &qmin, &qmax);
    if (st != TQ_OK) return st;
    TQ_REQUIRE(n >= 0, "%s: negative size", what);
    TQ_REQUIRE(scale_zp && workspace, "%s: null scale_zp/workspace", what);
    TQ_REQUIRE(n == 0 || (x && q), "%s: null pointer", what);
    TQ_REQUIRE(aligned(workspace, 16) && aligned(scale_zp, 8), "%s: misaligned workspace/scale_zp", what);
    const hipStream_t s = as_hip(stream);
    using K = typename OrderedKey<T>::K;
    K* ws = static_cast<K*>(workspace);
    k_per_tensor_init<T><<<1, kWave, 0, s>>>(ws);
    if (n > 0) k_minmax_keys<T><<<grid_for(n, kBlock * 8, 4096), kBlock, 0, s>>>(x, n, ws);
    k_per_tensor_quantize<T><<<grid_for(n, kBlock, 65536), kBlock, 0, s>>>(x, n, ws, qmin, qmax, q, scale_zp);
    return check_launch(what);
}

template <typename T>
int minmax_reset_impl(T* state, int64_t channels, tq_stream_t stream, const char* what) {
    TQ_REQUIRE(state && channels > 0, "%s: null state or channels <= 0", what);
    k_minmax_reset<T><<<grid_for(channels, kBlock, INT32_MAX), kBlock, 0, as_hip(stream)>>>(state, channels);
    return check_launch(what);
}

template <typename T>
int minmax_observe_impl(const T* x, int64_t n, T* state, tq_stream_t stream, const char* what) {
    TQ_REQUIRE(n >= 0 && state, "%s: bad arguments", what);
    if (n == 0) return TQ_OK;
    TQ_REQUIRE(x && aligned(state, sizeof(T)), "%s: null/misaligned pointer", what);
    k_minmax_observe<T><<<grid_for(n, kBlock * 8, 4096), kBlock, 0, as_hip(stream)>>>(x, n, state);
    return check_launch(what);
}

template <typename T>
int minmax_observe_per_channel_impl(const T* x, int64_t n, int64_t channels, T* state, tq_stream_t stream,
                                    const char* what) {
    TQ_REQUIRE(n >= 0 && channels > 0 && state, "%s: bad arguments", what);
    TQ_REQUIRE(channels < (int64_t(1) << 31), "%s: too many channels", what);
    const int64_t per = n / channels;
    if (per == 0) return TQ_OK;
    TQ_REQUIRE(x, "%s: null input", what);
    k_minmax_observe_per_channel<T><<<static_cast<unsigned>(channels), kBlock, 0, as_hip(stream)>>>(x, per, state);
    return check_launch(what);
}

}  // namespace
}  // namespace tq

extern "C" {

int tq_quantize_tensor(const float* x, int64_t n, double scale, double zero_point, int qdtype, float* q,
                       tq_stream_t stream) {
    return quantize_tensor_impl(x, n, scale, zero_point, qdtype, q, stream, "tq_quantize_tensor");
}
int tq_quantize_tensor_f64(const double* x, int64_t n, double scale, double zero_point, int qdtype, double* q,
                           tq_stream_t stream) {
    return quantize_tensor_impl(x, n, scale, zero_point, qdtype, q, stream, "tq_quantize_tensor_f64");
}

int tq_dequantize_tensor(const float* q, int64_t n, double scale, double zero_point, float* out,
                         tq_stream_t stream) {
    return dequantize_tensor_impl(q, n, scale, zero_point, out, stream, "tq_dequantize_tensor");
}
int tq_dequantize_tensor_f64(const double* q, int64_t n, double scale, double zero_point, double* out,
                             tq_stream_t stream) {
    return dequantize_tensor_impl(q, n, scale, zero_point, out, stream, "tq_dequantize_tensor_f64");
}

int tq_fake_quantize(const float* x, int64_t n, double scale, double zero_point, int qdtype, float* out,
                     tq_stream_t stream) {
    return fake_quantize_impl(x, n, scale, zero_point, qdtype, out, stream, "tq_fake_quantize");
}
int tq_fake_quantize_f64(const double* x, int64_t n, double scale, double zero_point, int qdtype, double* out,
                         tq_stream_t stream) {
    return fake_quantize_impl(x, n, scale, zero_point, qdtype, out, stream, "tq_fake_quantize_f64");
}

int tq_quantize_per_tensor(const float* x, int64_t n, int qdtype, float* q, double* scale_zp, void* workspace,
                           tq_stream_t stream) {
    return quantize_per_tensor_impl(x, n, qdtype, q, scale_zp, workspace, stream, "tq_quantize_per_tensor");
}
int tq_quantize_per_tensor_f64(const double* x, int64_t n, int qdtype, double* q, double* scale_zp,
                               void* workspace, tq_stream_t stream) {
    return quantize_per_tensor_impl(x, n, qdtype, q, scale_zp, workspace, stream, "tq_quantize_per_tensor_f64");
}

int tq_minmax_reset(float* state, int64_t channels, tq_stream_t stream) {
    return minmax_reset_impl(state, channels, stream, "tq_minmax_reset");
}
int tq_minmax_reset_f64(double* state, int64_t channels, tq_stream_t stream) {
    return minmax_reset_impl(state, channels, stream, "tq_minmax_reset_f64");
}

int tq_minmax_observe(const float* x, int64_t n, float* state, tq_stream_t stream) {
    return minmax_observe_impl(x, n, state, stream, "tq_minmax_observe");
}
int tq_minmax_observe_f64(const double* x, int64_t n, double* state, tq_stream_t stream) {
    return minmax_observe_impl(x, n, state, stream, "tq_minmax_observe_f64");
}

int tq_minmax_observe_per_channel(const float* x, int64_t n, int64_t channels, float* state,
                                  tq_stream_t stream) {
    return minmax_observe_per_channel_impl(x, n, channels, state, stream, "tq_minmax_observe_per_channel");
}
int tq_minmax_observe_per_channel_f64(const double* x, int64_t n, int64_t channels, double* state,
                                      tq_stream_t stream) {
    return minmax_observe_per_channel_impl(x, n, channels, state, stream, "tq_minmax_observe_per_channel_f64");
}

}  // extern "C"
