/*
 * tq.h -- C ABI of the MI355X (gfx950) quantized-inference library libtq.so.
 *
 * This is the drop-in boundary for neo-theano's `theano-quantize` crate: the
 * entry points below are what the theano-rocm FFI layer binds (an
 * `extern "C"` block on the Rust side) to run the crate's quantize,
 * dequantize and quantized-Linear work on the GPU.  Each declaration names
 * the reference interface it replaces (paths relative to the reference
 * repository root).
 *
 * Conventions (all entry points):
 *  - every tensor pointer is caller-owned DEVICE memory, row-major, dense;
 *  - `stream` is the last argument; work is enqueued asynchronously on it and
 *    is stream-ordered.  NULL means the default stream;
 *  - the library allocates nothing and keeps no mutable global state, so calls
 *    on distinct streams are reentrant and thread-safe (one exception:
 *    tq_mlp_w4g128_decode_noalloc's per-device scratch, see there);
 *  - integer sizes are int64_t; a size of zero is a valid no-op unless noted;
 *  - the return value is a tq_status.  On failure nothing was enqueued and
 *    tq_last_error() (thread-local) holds a message.  The statuses map onto
 *    the reference's error types: TQ_EINVAL -> TheanoError::InvalidArgument /
 *    ShapeMismatch (crates/theano-types/src/error.rs:7-56), TQ_EHIP ->
 *    RocmError::KernelError / DriverError, TQ_ENOMEM -> RocmError::OutOfMemory
 *    (crates/theano-rocm/src/error.rs:3-73).
 *
 * Numerics (the parity contract):
 *  - codes use the reference rounding, round-half-away-from-zero of the exact
 *    quotient x/scale (+ zero point), then clamp (quantize.rs:15); integer
 *    codes, packed bytes, scales and int32 accumulators are bit-exact with the
 *    reference CPU path; dequantized values are bit-exact (IEEE ==, the
 *    reference's -0.0 codes become +0.0);
 *  - a NaN input gives code 0 (Rust's `f64 as i8` of the reference's NaN code);
 *  - float matmul outputs are f32 with f32 accumulation, within 1e-3 relative
 *    / 1e-4 absolute of the reference's f64 result.
 */
#ifndef TQ_H
#define TQ_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* tq_stream_t; /* hipStream_t */

typedef enum {
    TQ_OK = 0,
    TQ_EINVAL = 1,  /* bad shape, pointer, alignment or argument */
    TQ_EHIP = 2,    /* HIP runtime / launch failure */
    TQ_ENOMEM = 3,  /* device allocation failure (host-side helpers only) */
} tq_status;

/* DType of a device buffer: crates/theano-types/src/dtype.rs:5-25 (same order;
 * complex and quantized variants have no element conversion here). */
typedef enum {
    TQ_DT_F16 = 0,
    TQ_DT_BF16 = 1,
    TQ_DT_F32 = 2,
    TQ_DT_F64 = 3,
    TQ_DT_U8 = 4,
    TQ_DT_I8 = 5,
    TQ_DT_I16 = 6,
    TQ_DT_I32 = 7,
    TQ_DT_I64 = 8,
    TQ_DT_BOOL = 9,
} tq_dtype;

/* QuantDType: crates/theano-quantize/src/qconfig.rs:5-10 (same order) */
typedef enum {
    TQ_QINT8 = 0,
    TQ_QUINT8 = 1,
    TQ_QINT4 = 2,
    TQ_QFP8 = 3, /* range +-448 only, as in the reference (no FP8 encoding) */
} tq_qdtype;

/* Library version (major*10000 + minor*100 + patch). */
int tq_version(void);
/* Human-readable name of a status. */
const char* tq_status_string(int status);
/* Message describing the last failure on the calling thread ("" if none). */
const char* tq_last_error(void);

/* QuantDType::{bits, is_signed, qmin, qmax}: qconfig.rs:12-41. Host-only. */
int tq_qdtype_info(int qdtype, int* bits, int* is_signed, double* qmin, double* qmax);

/* ------------------------------------------------------------------------
 * Reference primitives on device data.
 * Codes are returned as f32 values: every code the reference returns in its
 * Vec<f64> (integral, within +-448, -0.0 and NaN included) is exactly
 * representable in f32, so the f32 buffer holds the reference's codes
 * bit-for-bit after widening.  Arithmetic is done in f64 on the GPU.
 * Each primitive also has an _f64 form with f64 data in and out (the
 * reference's own element type: Tensor storage and Vec<f64>), which returns
 * exactly the reference's f64 results for any f64 input; the f32 forms are
 * the device-native ones for f32 tensors.
 * ------------------------------------------------------------------------ */

/* quantize_tensor (crates/theano-quantize/src/quantize.rs:8-19):
 *   q[i] = clamp(round(x[i]/scale + zero_point), qmin, qmax) */
int tq_quantize_tensor(const float* x, int64_t n, double scale, double zero_point,
                       int qdtype, float* q, tq_stream_t stream);
int tq_quantize_tensor_f64(const double* x, int64_t n, double scale, double zero_point,
                           int qdtype, double* q, tq_stream_t stream);

/* dequantize_tensor (quantize.rs:22-27): out[i] = f32((q[i] - zero_point) * scale) */
int tq_dequantize_tensor(const float* q, int64_t n, double scale, double zero_point,
                         float* out, tq_stream_t stream);
/* out[i] = (q[i] - zero_point) * scale in f64 (the reference's Vec<f64> result) */
int tq_dequantize_tensor_f64(const double* q, int64_t n, double scale, double zero_point,
                             double* out, tq_stream_t stream);

/* fake_quantize (quantize.rs:51-55): out = f32(dequantize(quantize(x))) */
int tq_fake_quantize(const float* x, int64_t n, double scale, double zero_point,
                     int qdtype, float* out, tq_stream_t stream);
int tq_fake_quantize_f64(const double* x, int64_t n, double scale, double zero_point,
                         int qdtype, double* out, tq_stream_t stream);

/* quantize_per_tensor (quantize.rs:30-48): asymmetric scale/zero point from the
 * data's min/max, then quantize_tensor.  scale_zp (device, 2 doubles) receives
 * {scale, zero_point}.  workspace: device memory of TQ_PER_TENSOR_WORKSPACE
 * bytes, 16-byte aligned, contents need not be initialised. */
#define TQ_PER_TENSOR_WORKSPACE 64
int tq_quantize_per_tensor(const float* x, int64_t n, int qdtype, float* q,
                           double* scale_zp, void* workspace, tq_stream_t stream);
int tq_quantize_per_tensor_f64(const double* x, int64_t n, int qdtype, double* q,
                               double* scale_zp, void* workspace, tq_stream_t stream);

/* MinMaxObserver::{reset, observe} (crates/theano-quantize/src/observer.rs:42-73).
 * state (device, 2 floats) = {min, max}; reset sets {+inf, -inf}; observe
 * folds min/max ignoring NaN.  compute_scale_zero_point is scalar host math
 * (see tq_observer_scale_zp). */
int tq_minmax_reset(float* state, int64_t channels, tq_stream_t stream);
int tq_minmax_observe(const float* x, int64_t n, float* state, tq_stream_t stream);
/* the same with f64 values and an f64 state (channels x {min, max} doubles) */
int tq_minmax_reset_f64(double* state, int64_t channels, tq_stream_t stream);
int tq_minmax_observe_f64(const double* x, int64_t n, double* state, tq_stream_t stream);

/* PerChannelMinMaxObserver::observe (observer.rs:110-121): values laid out
 * [channels, n/channels] (a trailing remainder is ignored, as in the
 * reference); state (device) = channels x {min, max}. */
int tq_minmax_observe_per_channel(const float* x, int64_t n, int64_t channels,
                                  float* state, tq_stream_t stream);
int tq_minmax_observe_per_channel_f64(const double* x, int64_t n, int64_t channels,
                                      double* state, tq_stream_t stream);

/* compute_scale_zero_point for one {min,max} pair (observer.rs:51-66,93-106).
 * Host-only scalar helper; initialized=0 gives (1, 0) as the reference does. */
int tq_observer_scale_zp(double min_val, double max_val, int initialized, int qdtype,
                         double* scale, double* zero_point);

/* ------------------------------------------------------------------------
 * Weight formats (build-defined compositions of the primitives above).
 * ------------------------------------------------------------------------ */

/* Symmetric per-row INT8 (per output channel for a [N, K] weight; per token
 * for [M, K] activations):
 *   s[r] = f32(max(absmax_r / 127, 1e-10)),  absmax from the observer's
 *          min/max (observer.rs:110-121) and the 1e-10 floor of quantize.rs:39
 *   q[r,k] = quantize_tensor(row r, f64(s[r]), 0, Int8)   (quantize.rs:8-19)
 * W [rows, K] f32 -> q int8 [rows, K], s f32 [rows]. */
int tq_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q, float* s,
                           tq_stream_t stream);
/* dequantize_tensor per row (quantize.rs:22-27): w_hat = f32(q * s[r]). */
int tq_dequantize_i8_rowwise(const int8_t* q, const float* s, int64_t rows, int64_t k,
                             float* w_hat, tq_stream_t stream);
/* Both in one pass (fake_quantize per row, quantize.rs:51-55); q, s, w_hat as above. */
int tq_fake_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q,
                                float* s, float* w_hat, tq_stream_t stream);

/* Symmetric per-row FP8, OCP E4M3 (bias 7, largest finite 448, S.1111.111 =
 * NaN): the 8-bit float behind QuantDType::FP8, whose range the reference
 * states as [-448, 448] (qconfig.rs:29,38) without an encoding.
 *   s[r]   = f32(max(absmax_r / 448, 1e-10))   (absmax as for INT8 above)
 *   q[r,k] = e4m3_rne(clamp(f32(w[r,k] / s[r]), -448, 448)),  NaN -> 0x7F
 * W [rows, K] f32 -> q u8 [rows, K] (e4m3 bit patterns), s f32 [rows]. */
int tq_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q, float* s,
                            tq_stream_t stream);
/* w_hat = f32(e4m3(q) * s[r]) (one rounding of an exact product). */
int tq_dequantize_fp8_rowwise(const uint8_t* q, const float* s, int64_t rows, int64_t k,
                              float* w_hat, tq_stream_t stream);
/* Both in one pass (fake_quantize per row with the FP8 grid). */
int tq_fake_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q,
                                 float* s, float* w_hat, tq_stream_t stream);

/* Symmetric INT4 with groups of 128 along K (K % 128 == 0):
 *   s[r,g] = max(f16_rne(absmax_{r,g} / 7), 2^-24)   (f16 bits)
 *   q      = quantize_tensor(group, f64(s), 0, Int4)  in [-8, 7]
 *   packed[r, j] = (q[r,2j] & 0xF) | (q[r,2j+1] & 0xF) << 4   (low nibble = even k)
 * W [rows, K] f32 -> packed u8 [rows, K/2], s f16 [rows, K/128]. */
int tq_quantize_i4_g128(const float* w, int64_t rows, int64_t k, uint8_t* packed,
                        uint16_t* s_f16, tq_stream_t stream);
/* w_hat = f32(q * s) (exact). */
int tq_dequantize_i4_g128(const uint8_t* packed, const uint16_t* s_f16, int64_t rows,
                          int64_t k, float* w_hat, tq_stream_t stream);

/* ------------------------------------------------------------------------
 * Quantized Linear: y = x . dequant(W)^T (+ bias), the reference's
 * Linear::forward (crates/theano-nn/src/linear.rs:111-121) over the
 * dequantized weight that Linear::from_tensors receives (linear.rs:65-75).
 * y is f32 [M, N]; bias (f32 [N]) may be NULL.
 * ------------------------------------------------------------------------ */

/* Decode-shaped GEMV, INT8 per-row weights, f32 activations x [M, K], M <= 16
 * (longer inputs run in chunks of 16 rows).  Any N, K; f32 pointers 4-byte
 * aligned.  The tuned kernel serves K % 16 == 0, K <= 8192 with x and q 16-byte
 * aligned; other shapes take a shape-general kernel. */
int tq_gemv_w8(const float* x, int64_t m, const int8_t* q, const float* s,
               const float* bias, int64_t n, int64_t k, float* y, tq_stream_t stream);

/* The same GEMV over per-row FP8 (OCP e4m3) weights (tq_quantize_fp8_rowwise):
 * y = s[n] * sum_k e4m3(q[n,k]) * x[m,k] (+ bias[n]), f32 accumulation.  Same
 * shapes, alignment and kernels as tq_gemv_w8. */
int tq_gemv_fp8(const float* x, int64_t m, const uint8_t* q, const float* s,
                const float* bias, int64_t n, int64_t k, float* y, tq_stream_t stream);

/* Decode-shaped W8A8 with the activation quantization fused in: x f32 [M, K],
 * M <= 16, is quantized per row inside the kernel exactly as
 * tq_quantize_i8_rowwise does, then y = fma(f32(sum_p qa*qw) * sa, sw, bias)
 * with exact int32 dot products: the same y as tq_quantize_i8_rowwise +
 * tq_gemm_w8a8, bit for bit, in one launch.  Requires K % 16 == 0, K <= 8192,
 * x and qw 16-byte aligned (TQ_EINVAL otherwise: run the two-step path).  At
 * 4096 x 4096 faster than the two-step path for M <= 2 (5.1 against 9.2-9.5 us
 * at M = 1), slower from M = 3 (13.3 against 9.7-9.9 us at 4; 49.4 against 11.3
 * at 16). */
int tq_gemv_w8a8(const float* x, int64_t m, const int8_t* qw, const float* sw,
                 const float* bias, int64_t n, int64_t k, float* y, tq_stream_t stream);
/* The FP8 counterpart (tq_quantize_fp8_rowwise + tq_gemm_fp8 in one launch;
 * f32 accumulation, so equal to the GEMM within the float tolerance).  Faster
 * than the two-step path at 4096 x 4096 for M <= 2 (5.5-5.6 against 9.3-9.5 us
 * at M = 1), slower from M = 3 (12.9 against 10.0 us; 54.0 against 11.3 at 16). */
int tq_gemv_fp8a8(const float* x, int64_t m, const uint8_t* qw, const float* sw,
                  const float* bias, int64_t n, int64_t k, float* y, tq_stream_t stream);

/* Decode-shaped GEMV, INT4 g128 weights (canonical layout), bf16 activations
 * x [M, K] (bf16 bits), M <= 16, K % 128 == 0 (the format), any N.  The MFMA
 * kernel serves K <= 16384 with x and packed 16-byte aligned; other cases take
 * a shape-general kernel. */
int tq_gemv_w4g128(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                   const uint16_t* s_f16, const float* bias, int64_t n, int64_t k,
                   float* y, tq_stream_t stream);

/* Row-tiled kernel layout of an INT4 g128 weight for the decode GEMV (a pure
 * permutation of the canonical bytes; rows padded to a multiple of tile_rows
 * with zero bytes and zero scales).  With C = K/32 16-byte chunks per row,
 * G = K/128 groups and T = tile_rows:
 *   packed_t[((t*C + c)*T + r)*16 + b] = packed[t*T + r][16c + b]
 *   s_t[(t*G + g)*T + r]               = s[t*T + r][g]
 * Buffer sizes: packed_t ceil(N/T)*T*K/2 bytes, s_t ceil(N/T)*T*K/128 halves.
 * tq_w4g128_tile_rows picks T (a multiple of 8 in [8, 64]) so that the tiles
 * about match the compute units of the current device (host-only). */
int64_t tq_w4g128_tile_rows(int64_t n);
int tq_repack_w4g128_tiled(const uint8_t* packed, const uint16_t* s_f16, int64_t n, int64_t k,
                           int64_t tile_rows, uint8_t* packed_t, uint16_t* s_t, tq_stream_t stream);
/* Decode-shaped GEMV on the tiled layout: same result as tq_gemv_w4g128.
 * M <= 16, K % 128 == 0, K <= 16384. */
int tq_gemv_w4g128_tiled(const uint16_t* x_bf16, int64_t m, const uint8_t* packed_t,
                         const uint16_t* s_t, const float* bias, int64_t n, int64_t k,
                         int64_t tile_rows, float* y, tq_stream_t stream);

/* Prefill-shaped W8A8: activations already quantized per row (use
 * tq_quantize_i8_rowwise on X).  acc[i,j] = sum_p qa[i,p]*qw[j,p] (int32,
 * bit-exact); y = fma(f32(acc) * sa[i], sw[j], bias[j] or 0).  acc may be NULL.
 * Any M, N, K.  The MFMA kernels serve N % 16 == 0 and K % 16 == 0 (M <= 16 with
 * K % 64 == 0 and K <= 8192: a skinny kernel of N/16 blocks, 16 weight rows each;
 * the LDS-DMA kernel K % 128 == 0) with 16-byte aligned qa, qw, sw, bias, y and
 * acc; other cases take a shape-general kernel. */
int tq_gemm_w8a8(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                 const float* bias, int64_t m, int64_t n, int64_t k, int32_t* acc,
                 float* y, tq_stream_t stream);

/* Prefill-shaped FP8 W8A8 (both operands per-row E4M3, tq_quantize_fp8_rowwise):
 * y[i,j] = fma(f32(sum_p e4m3(qa[i,p]) * e4m3(qw[j,p])) * sa[i], sw[j], bias[j] or 0);
 * products exact, f32 accumulation.  The reference value is Linear over the
 * dequantized operands (linear.rs:111-121, tensor_ops.rs:379-410).  Any M, N,
 * K.  The FP8 MFMA kernels serve K % 128 == 0 and N % 16 == 0 with 16-byte
 * aligned qa, qw, sw, bias and y (M <= 16 with K <= 8192: a skinny kernel of N/16
 * blocks); other cases take a shape-general kernel. */
int tq_gemm_fp8(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                const float* bias, int64_t m, int64_t n, int64_t k, float* y, tq_stream_t stream);

/* Prefill-shaped W4A16: x bf16 [M, K], INT4 g128 weights, f32 accumulation with
 * the group scale applied to each 128-long partial sum; y f32 [M, N].
 * K % 128 == 0 (the format), any M, N.  The MFMA kernel serves N % 16 == 0 with
 * 16-byte aligned x, packed, y and bias; other cases take a shape-general kernel. */
int tq_gemm_w4g128_bf16(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                        const uint16_t* s_f16, const float* bias, int64_t n, int64_t k,
                        float* y, tq_stream_t stream);

/* The same Linear (crates/theano-nn/src/linear.rs:111-121 over the dequantized
 * weight) on the pipelined FFN kernels: x in the kernels' k-order and
 * its group sums go to `workspace` (at least
 * tq_gemm_w4g128_bf16_workspace_bytes(M, K) bytes, 256-byte aligned).  Runs when
 * K % 256 == 0 and N % 256 == 0 with 16-byte aligned x, packed and y and
 * 4-byte aligned scales; other shapes take tq_gemm_w4g128_bf16.  When twice
 * the output tiles still fit the CUs in one round, K is split in two halves
 * added into y (zeroed first; two addends onto zero, so the result is
 * deterministic). */
int64_t tq_gemm_w4g128_bf16_workspace_bytes(int64_t m, int64_t k);
int tq_gemm_w4g128_bf16_ws(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                           const uint16_t* s_f16, const float* bias, int64_t n, int64_t k,
                           void* workspace, int64_t workspace_bytes, float* y,
                           tq_stream_t stream);

/* Quantized Llama-style FFN (build-defined composition of Linear, SiLU
 * (crates/theano-nn/src/activation.rs:66-79) and Tensor::mul):
 *   h = SiLU(x Wg^T) * (x Wu^T);   y = h Wd^T   (f32 [M, D]).
 * x bf16 [M, D]; gate/up INT4 g128 [F, D]; down INT4 g128 [D, F];
 * D % 128 == 0, F % 128 == 0.  `workspace` is device memory of at least
 * tq_mlp_w4g128_workspace_bytes(M, D, F) bytes (intermediates: x in the
 * kernels' k-order, h as bf16 hi + lo planes, group sums; or h as f32 [M, F]
 * on the shape-general path), 16-byte aligned; the pipelined kernels run when
 * D % 256 == 0, F % 256 == 0, the workspace is 256-byte aligned and the
 * scales 4-byte aligned.  x, packed weights and y 16-byte aligned. */
int64_t tq_mlp_w4g128_workspace_bytes(int64_t m, int64_t d, int64_t f);
int tq_mlp_w4g128(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                  const uint8_t* gate_packed, const uint16_t* gate_s,
                  const uint8_t* up_packed, const uint16_t* up_s,
                  const uint8_t* down_packed, const uint16_t* down_s,
                  void* workspace, int64_t workspace_bytes, float* y, tq_stream_t stream);

/* The same FFN for decode shapes (M <= 16; at D = 4096, F = 14336 faster than
 * tq_mlp_w4g128 at every such M: 35-60 against 134-136 us at M = 5-16) on
 * row-tiled copies of the weights (permutations of the packed bytes):
 *   gate and up:  tq_repack_w4g128_gate_up_tiled -> 64-row tiles, tile t holding
 *                 gate rows 32t..32t+31 then up rows 32t..32t+31, padded to F
 *                 rounded up to 32 with zeros ((F+31)/32 * 64 * D/2 bytes and
 *                 (F+31)/32 * 64 * D/128 scales);
 *   down:         tq_repack_w4g128_tiled with tile_rows 16, 32 or 64; 32 (the
 *                 host layers' choice) runs one launch per four tokens with
 *                 K split over two blocks per tile, 2 * D / 32 blocks.
 * h = SiLU(x Wg^T) * (x Wu^T) is formed in f32 per token and handed to the down
 * projection as bf16 hi + lo (lo = bf16(h - hi)).  D, F multiples of 128 and at
 * most 16384.  `workspace`: tq_mlp_w4g128_decode_workspace_bytes(M, D, F)
 * bytes, 16-byte aligned; x and the scales 8-byte aligned, packed weights
 * 16-byte aligned.  These three have no counterpart in the reference: they
 * serve its FFN composition (Linear, SiLU, Tensor::mul) at decode batch sizes. */
int64_t tq_mlp_w4g128_decode_workspace_bytes(int64_t m, int64_t d, int64_t f);
int tq_repack_w4g128_gate_up_tiled(const uint8_t* gate_packed, const uint16_t* gate_s,
                                   const uint8_t* up_packed, const uint16_t* up_s, int64_t f, int64_t d,
                                   uint8_t* packed_t, uint16_t* s_t, tq_stream_t stream);
int tq_mlp_w4g128_decode(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                         const uint8_t* gate_up_t, const uint16_t* gate_up_s_t,
                         const uint8_t* down_t, const uint16_t* down_s_t, int64_t down_tile_rows,
                         void* workspace, int64_t workspace_bytes, float* y, tq_stream_t stream);

/* The decode FFN above with no workspace argument and no allocation, for
 * callers that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc).  It has no counterpart in
 * the reference.  h (and its block sums) lives in a scratch array inside
 * libtq.so, one per device, of TQ_MLP_DECODE_SCRATCH_BYTES (16 tokens at
 * F = 16384), held until the process ends; shapes needing more
 * (tq_mlp_w4g128_decode_workspace_bytes) are rejected with TQ_EINVAL.  The result equals tq_mlp_w4g128_decode's bit for
 * bit.  Every call on one device shares that device's scratch, so calls that
 * overlap in time on one device (distinct streams, or distinct threads without
 * ordering) race and give undefined results; calls ordered on one stream are
 * safe.  The first call on a device resolves the scratch address once
 * (thread-safe); nothing is allocated. */
#define TQ_MLP_DECODE_SCRATCH_BYTES ((1 << 20) + (1 << 16))
int tq_mlp_w4g128_decode_noalloc(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                                 const uint8_t* gate_up_t, const uint16_t* gate_up_s_t,
                                 const uint8_t* down_t, const uint16_t* down_s_t,
                                 int64_t down_tile_rows, float* y, tq_stream_t stream);

/* ------------------------------------------------------------------------
 * Attention core of MultiheadAttention::forward_with_mask
 * (crates/theano-nn/src/transformer.rs:95-142) between the quantized q/k/v and
 * out projections, f32:
 *   scores = (Q_h K_h^T) * (1/sqrt(head_dim)) (+ mask);  P = softmax(scores, -1)
 *   (tensor_ops.rs:574-620);  O_h = P V_h, heads concatenated.
 * q, k, v: [batch * seq, ld*] row-major, head h in columns [h*D, (h+1)*D)
 * (the fused QKV projection's [B*S, 3E] output in place: ld = 3E, k = q + E,
 * v = q + 2E).  mask: NULL (mask_batch = 0) or additive f32 [mask_batch, seq,
 * seq], mask_batch 1 (broadcast) or batch, shared by the heads.  out: [batch *
 * seq, ldo].  head_dim <= 128.  A row whose scores are all -inf gives NaN, as
 * the reference's softmax does.  head_dim % 4 == 0 with k and v 16-byte aligned
 * and ldk, ldv multiples of 4 takes the faster quad-load kernel; every form
 * gives the same bits.
 * ------------------------------------------------------------------------ */
int tq_attention_f32(const float* q, int64_t ldq, const float* k, int64_t ldk, const float* v,
                     int64_t ldv, const float* mask, int64_t mask_batch, int64_t batch, int64_t seq,
                     int64_t heads, int64_t head_dim, float* out, int64_t ldo, tq_stream_t stream);

/* ------------------------------------------------------------------------
 * Element type conversion of device buffers: the device half of Tensor::to
 * (crates/theano-core/src/tensor.rs:277-299) and of RocmStorage::from_host_f64
 * / to_host_f64 (crates/theano-rocm/src/storage.rs:54-99), whose tensors hold
 * f64 values in a buffer of their DType.
 * dst[i] = cast(f64(src[i])): F32/F16/BF16 round to nearest even from the f64
 * value (overflow -> inf, NaN stays NaN); integer types follow Rust's
 * `f64 as T` (toward zero, saturating, NaN -> 0); Bool is value != 0.
 * src and dst must not overlap and are aligned to their element sizes.
 * ------------------------------------------------------------------------ */
int64_t tq_dtype_size(int dtype); /* bytes per element, 0 if unsupported */
int tq_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n,
               tq_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* TQ_H */
