// tq_internal.h -- shared host/device helpers of libtq.so (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>

#include "../../include/tq.h"

namespace tq {

// Native clang vectors (HIP's float4 & co. are structs, which the
// nontemporal and bit-cast builtins do not accept).
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------- host side

// Records a thread-local error message and returns `status`.
int fail(int status, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline hipStream_t as_hip(tq_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Checks the launch that was just enqueued.
int check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// Compute-unit count of the current device (cached per device, thread-safe).
int device_cu_count();

// Raises `kernel`'s dynamic LDS limit to `bytes` once per device (bit d of
// `done_devices` records device d); thread-safe.
int allow_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done_devices);

// Shape-general fallbacks of the matmul entry points (tq_generic.hip); any N,
// K (K % 128 == 0 for INT4 g128), element-aligned pointers.
int launch_linear_8bit_generic(const float* x, int64_t m, const int8_t* q, const float* s, const float* bias,
                               int64_t n, int64_t k, float* y, hipStream_t st);
int launch_linear_8bit_generic(const float* x, int64_t m, const uint8_t* q, const float* s, const float* bias,
                               int64_t n, int64_t k, float* y, hipStream_t st);
int launch_linear_w4_generic(const uint16_t* x, int64_t m, const uint8_t* packed, const uint16_t* s16,
                             const float* bias, int64_t n, int64_t k, float* y, hipStream_t st);
int launch_gemm_w8a8_generic(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                             const float* bias, int64_t m, int64_t n, int64_t k, int32_t* acc, float* y,
                             hipStream_t st);
int launch_gemm_fp8_generic(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                            const float* bias, int64_t m, int64_t n, int64_t k, float* y, hipStream_t st);

// FFN block for shapes the pipelined kernels of tq_ffn.hip do not take (D or F
// not a multiple of 256, 2-byte aligned scales): 16x16x32 MFMA kernels of
// tq_mlp.hip with h kept as f32 [M, F] in `h`.
int launch_mlp_w4g128_general(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f, const uint8_t* gate_packed,
                              const uint16_t* gate_s, const uint8_t* up_packed, const uint16_t* up_s,
                              const uint8_t* down_packed, const uint16_t* down_s, float* h, float* y,
                              hipStream_t st);

#define TQ_REQUIRE(cond, ...)                                 \
    do {                                                      \
        if (!(cond)) return ::tq::fail(TQ_EINVAL, __VA_ARGS__); \
    } while (0)

// -------------------------------------------------------------- device side

constexpr int kWave = 64;

typedef __attribute__((address_space(3))) int8_t lds_i8;

// LDS byte address (the low 32 bits of an LDS pointer; an address-space cast).
__device__ __forceinline__ uint32_t lds_addr(const int8_t* l) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_i8*)l));
}

// Direct global -> LDS loads: each active lane's bytes at `g` land at
// la + lane * size (M0 holds the wave's LDS base).  These are the only writers
// of M0 in the library.  Issued as inline asm because the compiler cannot tell
// which LDS buffer a pending LDS DMA targets and would otherwise wait for all of
// them before every LDS read; callers track completion with explicit vmcnt
// waits.  M0 is listed as clobbered so that the compiler never assumes a value
// of its own survives the statement (clang warns that M0 is reserved, i.e. not
// saved for the statement, which is the intent: nothing is to be preserved).
// An LDS DMA reads M0 one wait state after a scalar write of it (the gap the
// compiler itself leaves between the two on gfx950), hence the s_nop 0: the
// hazard recognizer does not look inside inline asm.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void lds_dma16(const void* g, uint32_t la) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(la), "v"(g) : "memory", "m0");
}
__device__ __forceinline__ void lds_dma4(const void* g, uint32_t la) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dword %1, off" ::"s"(la), "v"(g) : "memory", "m0");
}
// Waits until at most N vector memory operations of the wave are outstanding (the
// completion of LDS DMAs, which the compiler does not track).  A count N > 0 is
// only safe when every load it counts is issued by inline asm too: the compiler
// moves its own loads of restrict read-only memory across inline asm, memory
// clobber or not.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt counts 0..63");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
#pragma clang diagnostic pop

// Lane permutes within rows of 16 lanes through DPP, a VALU operand modifier
// (__shfl_xor compiles to ds_bpermute, a round trip through the LDS crossbar).
enum DppCtrl : int {
    kDppXor1 = 0xB1,         // quad_perm [1, 0, 3, 2]: lane i <- i ^ 1
    kDppXor2 = 0x4E,         // quad_perm [2, 3, 0, 1]: lane i <- i ^ 2
    kDppMirror = 0x140,      // lane i <- 15 - i within its row
    kDppHalfMirror = 0x141,  // lane i <- 7 - i within its half row
};
template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}
template <int kCtrl, class T>
__device__ __forceinline__ T dpp(T v) {
    static_assert(sizeof(T) == 4, "32-bit lanes");
    return __builtin_bit_cast(T, dpp_u32<kCtrl>(__builtin_bit_cast(uint32_t, v)));
}
template <class T>
__device__ __forceinline__ T readlane(T v, int l) {
    return __builtin_bit_cast(T, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

struct OpAdd {
    template <class T>
    __device__ T operator()(T a, T b) const { return a + b; }
};
struct OpMax {
    __device__ float operator()(float a, float b) const { return fmaxf(a, b); }
};
struct OpMin {
    __device__ float operator()(float a, float b) const { return fminf(a, b); }
};

// Reduction over each aligned group of kWidth (1, 2, 4, 8 or 16) lanes, in every
// lane of the group, for groups whose lanes are all active: quad butterflies,
// then the mirrored half row and the mirrored row bring in the other quad and
// the other half.
template <int kWidth, class T, class Op>
__device__ __forceinline__ T lane_group_reduce(T v, Op op) {
    static_assert(kWidth == 1 || kWidth == 2 || kWidth == 4 || kWidth == 8 || kWidth == 16,
                  "DPP groups are 1, 2, 4, 8 or 16 lanes");
    if constexpr (kWidth >= 2) v = op(v, dpp<kDppXor1>(v));
    if constexpr (kWidth >= 4) v = op(v, dpp<kDppXor2>(v));
    if constexpr (kWidth >= 8) v = op(v, dpp<kDppHalfMirror>(v));
    if constexpr (kWidth >= 16) v = op(v, dpp<kDppMirror>(v));
    return v;
}
template <int kWidth>
__device__ __forceinline__ float lane_group_sum(float v) {
    return lane_group_reduce<kWidth>(v, OpAdd{});
}
// Max over aligned groups of kWidth (1 to 16) lanes.
template <int kWidth>
__device__ __forceinline__ float group_max(float v) {
    return lane_group_reduce<kWidth>(v, OpMax{});
}

// Wave64 reductions with every lane active, result uniform: DPP within each
// 16-lane row, then the four rows' values (v_readlane) combined in a fixed
// order.  No LDS traffic (a __shfl_xor butterfly is six dependent ds_bpermute).
template <class T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
    v = lane_group_reduce<16>(v, op);
    return op(op(readlane(v, 0), readlane(v, 16)), op(readlane(v, 32), readlane(v, 48)));
}
__device__ __forceinline__ float wave_max(float v) { return wave_reduce(v, OpMax{}); }
__device__ __forceinline__ float wave_min(float v) { return wave_reduce(v, OpMin{}); }
__device__ __forceinline__ float wave_sum(float v) { return wave_reduce(v, OpAdd{}); }
__device__ __forceinline__ int wave_sum(int v) { return wave_reduce(v, OpAdd{}); }

// round_half_away_from_zero(a / s) for a >= 0 (or +inf), s > 0 finite normal,
// exact with respect to the real quotient (the reference rounds the f64
// quotient, which lies on the same side of every half-integer as the exact
// one).  `inv_s` is 1/s within 2 ulp; `cap` is an integer-valued float <= 256:
// quotients above cap come back as cap or cap+1, which every caller clamps.
// NaN `a` gives 0 (fmax(NaN, 0) = 0, and its NaN residual adds nothing).
//
// Why it is exact: for q = a/s <= cap + 1/2, t = fma(a, inv_s, 1/2 - 2^-12) is
// q + 1/2 - 2^-12 within q 2^-22 + 257 * 2^-24 < 2^-13, so n0 = floor(min(t,
// cap)) is the rounded n = floor(q + 1/2) or n - 1, never n + 1.  The residual
// r = fma(-n0, s, a), a - n0*s rounded once, decides: for n0 = n it is exact
// (|r| <= s/2 and, with a >= s/2, a multiple of ulp(s)/2; for a < s/2, n0 = 0
// and r = a) and below s/2; for n0 = n - 1 the exact value lies in [s/2, 1.5 s)
// and rounding keeps it >= s/2.  So n = n0 + 1 exactly when r >= s/2.  Above
// the cap, r > s/2 likewise.
__device__ __forceinline__ float rhaz_div(float a, float s, float inv_s, float half_s,
                                          float cap) {
    const float n = floorf(fminf(fmaxf(fmaf(a, inv_s, 0.5f - 0x1p-12f), 0.0f), cap));
    const float r = fmaf(-n, s, a);
    return (r >= half_s) ? n + 1.0f : n;
}

// Signed code for x given |x|'s rounded quotient n (rhaz_div: 0 for NaN x): sign
// from x, clamp to [qmin, qmax].
__device__ __forceinline__ int signed_code(float x, float n, int qmin, int qmax) {
    const int c = static_cast<int>(copysignf(n, x));  // n is integral, 0 <= n <= cap + 1
    return min(max(c, qmin), qmax);
}

}  // namespace tq
