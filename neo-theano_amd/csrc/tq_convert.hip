// tq_convert.hip -- element type conversion of device buffers, the device half
// of Tensor::to (crates/theano-core/src/tensor.rs:277-299) and of
// RocmStorage::from_host_f64 / to_host_f64
// (crates/theano-rocm/src/storage.rs:54-99).
//
// The reference keeps every tensor's values as f64 and records the DType
// beside them (Vec<f64> storage); a device buffer of DType d holds those values
// in d's element type.  A conversion is therefore defined on the f64 value:
//   dst = cast(f64(src)),
// with f64(src) exact for every source type except I64 (round to nearest even
// above 2^53), and cast:
//   F32, F16, BF16: round to nearest, ties to even, from the f64 value
//                   (overflow -> inf, NaN -> quiet NaN with the sign and the
//                   top payload bits);
//   I8 .. I64, U8:  Rust's `f64 as T`: toward zero, saturating, NaN -> 0;
//   Bool:           value != 0 (NaN -> 1).
// The float roundings work on the f64 bit pattern with integer arithmetic, so
// the result does not depend on the float rounding or denormal modes.
//
// HBM-bound: each thread converts 4 consecutive elements.
#include <limits>

#include "tq_internal.h"

namespace tq {
namespace {

constexpr int kBlock = 256;
constexpr int kPer = 4;

// f64 -> a binary format with kE exponent and kM mantissa bits, RNE.
template <int kE, int kM>
__device__ __forceinline__ uint32_t round_f64(double d) {
    const uint64_t b = __double_as_longlong(d);
    const uint32_t sign = static_cast<uint32_t>(b >> 63) << (kE + kM);
    const int e = static_cast<int>((b >> 52) & 0x7FF);
    const uint64_t m = b & ((uint64_t(1) << 52) - 1);
    constexpr uint32_t kExpAll = (1u << kE) - 1;
    constexpr int kBias = (1 << (kE - 1)) - 1;
    if (e == 0x7FF) {
        if (m == 0) return sign | (kExpAll << kM);                            // inf
        const uint32_t payload = static_cast<uint32_t>(m >> (52 - kM));      // top payload bits
        return sign | (kExpAll << kM) | (1u << (kM - 1)) | payload;          // quiet NaN
    }
    if (e == 0) return sign;  // f64 subnormal: far below half the target's smallest subnormal
    const uint64_t sig = m | (uint64_t(1) << 52);
    int E = e - 1023;
    int shift = 52 - kM;
    if (E < 1 - kBias) shift += (1 - kBias) - E;  // target subnormal range
    if (shift >= 54) return sign;                  // below half the smallest subnormal
    uint64_t q = sig >> shift;
    const uint64_t rem = sig & ((uint64_t(1) << shift) - 1), half = uint64_t(1) << (shift - 1);
    q += (rem > half || (rem == half && (q & 1))) ? 1 : 0;
    if (E < 1 - kBias) return sign | static_cast<uint32_t>(q);  // q == 2^kM is the smallest normal
    if (q == (uint64_t(1) << (kM + 1))) {
        q >>= 1;
        ++E;
    }
    const int biased = E + kBias;
    if (biased >= static_cast<int>(kExpAll)) return sign | (kExpAll << kM);  // overflow -> inf
    return sign | (static_cast<uint32_t>(biased) << kM) | static_cast<uint32_t>(q - (uint64_t(1) << kM));
}

// half / bfloat16 bits -> f64 (exact; a NaN keeps its sign and payload)
__device__ __forceinline__ double f16_value(uint16_t h) {
    const uint64_t sign = static_cast<uint64_t>(h & 0x8000) << 48;
    const int e = (h >> 10) & 0x1F, f = h & 0x3FF;
    if (e == 0x1F) return __longlong_as_double(sign | 0x7FF0000000000000ull | (static_cast<uint64_t>(f) << 42));
    const double mag = e == 0 ? ldexp(static_cast<double>(f), -24) : ldexp(static_cast<double>(f | 0x400), e - 25);
    return sign ? -mag : mag;
}

__device__ __forceinline__ double bf16_value(uint16_t h) {
    return static_cast<double>(__uint_as_float(static_cast<uint32_t>(h) << 16));
}

// Rust `f64 as T` for integers: toward zero, saturating, NaN -> 0
template <class T>
__device__ __forceinline__ T sat_int(double d) {
    constexpr double lo = static_cast<double>(std::numeric_limits<T>::min());
    constexpr double hi_excl = static_cast<double>(std::numeric_limits<T>::max()) + 1.0;  // 2^(bits-1) or 256
    if (!(d == d)) return T(0);
    if (d <= lo) return std::numeric_limits<T>::min();
    if (d >= hi_excl) return std::numeric_limits<T>::max();
    return static_cast<T>(d);
}

template <int kType> struct Elem;
template <> struct Elem<TQ_DT_F16> {
    typedef uint16_t T;
    __device__ static double get(T v) { return f16_value(v); }
    __device__ static T put(double d) { return static_cast<T>(round_f64<5, 10>(d)); }
};
template <> struct Elem<TQ_DT_BF16> {
    typedef uint16_t T;
    __device__ static double get(T v) { return bf16_value(v); }
    __device__ static T put(double d) { return static_cast<T>(round_f64<8, 7>(d)); }
};
template <> struct Elem<TQ_DT_F32> {
    typedef uint32_t T;
    __device__ static double get(T v) { return static_cast<double>(__uint_as_float(v)); }
    __device__ static T put(double d) { return round_f64<8, 23>(d); }
};
template <> struct Elem<TQ_DT_F64> {
    typedef double T;
    __device__ static double get(T v) { return v; }
    __device__ static T put(double d) { return d; }
};
template <> struct Elem<TQ_DT_U8> {
    typedef uint8_t T;
    __device__ static double get(T v) { return v; }
    __device__ static T put(double d) { return sat_int<uint8_t>(d); }
};
template <> struct Elem<TQ_DT_I8> {
    typedef int8_t T;
    __device__ static double get(T v) { return v; }
    __device__ static T put(double d) { return sat_int<int8_t>(d); }
};
template <> struct Elem<TQ_DT_I16> {
    typedef int16_t T;
    __device__ static double get(T v) { return v; }
    __device__ static T put(double d) { return sat_int<int16_t>(d); }
};
template <> struct Elem<TQ_DT_I32> {
    typedef int32_t T;
    __device__ static double get(T v) { return v; }
    __device__ static T put(double d) { return sat_int<int32_t>(d); }
};
template <> struct Elem<TQ_DT_I64> {
    typedef int64_t T;
    __device__ static double get(T v) { return static_cast<double>(v); }
    __device__ static T put(double d) { return sat_int<int64_t>(d); }
};
template <> struct Elem<TQ_DT_BOOL> {
    typedef uint8_t T;
    __device__ static double get(T v) { return v != 0 ? 1.0 : 0.0; }
    __device__ static T put(double d) { return d != 0.0 ? 1 : 0; }  // NaN != 0
};

template <int kSrc, int kDst>
__global__ __launch_bounds__(kBlock) void k_convert(const typename Elem<kSrc>::T* __restrict__ src,
                                                    typename Elem<kDst>::T* __restrict__ dst, int64_t n) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock * kPer;
    for (int64_t i0 = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * kPer; i0 < n; i0 += stride) {
        if (i0 + kPer <= n) {
            typename Elem<kSrc>::T v[kPer];
#pragma unroll
            for (int j = 0; j < kPer; ++j) v[j] = __builtin_nontemporal_load(src + i0 + j);
#pragma unroll
            for (int j = 0; j < kPer; ++j) dst[i0 + j] = Elem<kDst>::put(Elem<kSrc>::get(v[j]));
        } else {
            for (int64_t i = i0; i < n; ++i) dst[i] = Elem<kDst>::put(Elem<kSrc>::get(src[i]));
        }
    }
}

int elem_size(int t) {
    switch (t) {
        case TQ_DT_F16: case TQ_DT_BF16: case TQ_DT_I16: return 2;
        case TQ_DT_F32: case TQ_DT_I32: return 4;
        case TQ_DT_F64: case TQ_DT_I64: return 8;
        case TQ_DT_U8: case TQ_DT_I8: case TQ_DT_BOOL: return 1;
        default: return 0;
    }
}

template <int kSrc, int kDst>
void launch(const void* src, void* dst, int64_t n, unsigned grid, hipStream_t st) {
    k_convert<kSrc, kDst><<<grid, kBlock, 0, st>>>(static_cast<const typename Elem<kSrc>::T*>(src),
                                                   static_cast<typename Elem<kDst>::T*>(dst), n);
}

template <int kSrc>
bool dispatch_dst(int dst_t, const void* src, void* dst, int64_t n, unsigned grid, hipStream_t st) {
    switch (dst_t) {
        case TQ_DT_F16: launch<kSrc, TQ_DT_F16>(src, dst, n, grid, st); return true;
        case TQ_DT_BF16: launch<kSrc, TQ_DT_BF16>(src, dst, n, grid, st); return true;
        case TQ_DT_F32: launch<kSrc, TQ_DT_F32>(src, dst, n, grid, st); return true;
        case TQ_DT_F64: launch<kSrc, TQ_DT_F64>(src, dst, n, grid, st); return true;
        case TQ_DT_U8: launch<kSrc, TQ_DT_U8>(src, dst, n, grid, st); return true;
        case TQ_DT_I8: launch<kSrc, TQ_DT_I8>(src, dst, n, grid, st); return true;
        case TQ_DT_I16: launch<kSrc, TQ_DT_I16>(src, dst, n, grid, st); return true;
        case TQ_DT_I32: launch<kSrc, TQ_DT_I32>(src, dst, n, grid, st); return true;
        case TQ_DT_I64: launch<kSrc, TQ_DT_I64>(src, dst, n, grid, st); return true;
        case TQ_DT_BOOL: launch<kSrc, TQ_DT_BOOL>(src, dst, n, grid, st); return true;
        default: return false;
    }
}

bool dispatch(int src_t, int dst_t, const void* src, void* dst, int64_t n, unsigned grid, hipStream_t st) {
    switch (src_t) {
        case TQ_DT_F16: return dispatch_dst<TQ_DT_F16>(dst_t, src, dst, n, grid, st);
        case TQ_DT_BF16: return dispatch_dst<TQ_DT_BF16>(dst_t, src, dst, n, grid, st);
        case TQ_DT_F32: return dispatch_dst<TQ_DT_F32>(dst_t, src, dst, n, grid, st);
        case TQ_DT_F64: return dispatch_dst<TQ_DT_F64>(dst_t, src, dst, n, grid, st);
        case TQ_DT_U8: return dispatch_dst<TQ_DT_U8>(dst_t, src, dst, n, grid, st);
        case TQ_DT_I8: return dispatch_dst<TQ_DT_I8>(dst_t, src, dst, n, grid, st);
        case TQ_DT_I16: return dispatch_dst<TQ_DT_I16>(dst_t, src, dst, n, grid, st);
        case TQ_DT_I32: return dispatch_dst<TQ_DT_I32>(dst_t, src, dst, n, grid, st);
        case TQ_DT_I64: return dispatch_dst<TQ_DT_I64>(dst_t, src, dst, n, grid, st);
        case TQ_DT_BOOL: return dispatch_dst<TQ_DT_BOOL>(dst_t, src, dst, n, grid, st);
        default: return false;
    }
}

}  // namespace
}  // namespace tq

using namespace tq;

extern "C" int64_t tq_dtype_size(int dtype) { return elem_size(dtype); }

extern "C" int tq_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n, tq_stream_t stream) {
    TQ_REQUIRE(n >= 0, "tq_convert: negative length");
    const int ss = elem_size(src_dtype), ds = elem_size(dst_dtype);
    TQ_REQUIRE(ss > 0 && ds > 0, "tq_convert: unsupported dtype (src %d, dst %d)", src_dtype, dst_dtype);
    if (n == 0) return TQ_OK;
    TQ_REQUIRE(src && dst, "tq_convert: null pointer");
    TQ_REQUIRE(aligned(src, ss) && aligned(dst, ds), "tq_convert: pointer not aligned to its element size");
    const int64_t threads = (n + kPer - 1) / kPer;
    int64_t grid = (threads + kBlock - 1) / kBlock;
    const int64_t cap = static_cast<int64_t>(device_cu_count()) * 16;
    if (grid > cap) grid = cap;
    dispatch(src_dtype, dst_dtype, src, dst, n, static_cast<unsigned>(grid), as_hip(stream));
    return check_launch("tq_convert");
}
