/*
 * tq_oracle.h -- CPU restatement of neo-theano's quantized-inference path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * product path (libtq.so).  It is never linked into, loaded by or called from
 * the product; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may use it.
 *
 * Every function restates the reference's f64 arithmetic (Rust f64 is IEEE
 * binary64, round-to-nearest-even, no implicit FMA; this file is compiled with
 * -ffp-contract=off so C double arithmetic is bit-identical).  Rust
 * `f64::round` is C `round` (half away from zero), `f64::min/max` are
 * `fmin/fmax` (NaN-ignoring) and `f64::clamp` keeps NaN.
 *
 * Functions marked "build-defined" are compositions of the reference's
 * primitives that the reference itself does not ship (per-channel symmetric
 * INT8, INT4 group-128 packing, W8A8, the quantized MLP); their composition is
 * spelled out at each definition.
 *
 * Pinning status (what checks each function; details in tests/test_oracle.py):
 *   qdtype ranges          reference asserts qconfig.rs:82-108
 *   quantize_tensor        reference KAT quantize.rs:82-87, exact-rational ties
 *   dequantize_tensor      reference KAT quantize.rs:89-99
 *   quantize_per_tensor    reference tests quantize.rs:61-72,101-119,128-136,
 *                          brute force over the zero point
 *   observers              reference tests observer.rs:142-223
 *   mm / linear            reference KATs tensor_ops.rs:841-859, exact
 *                          integer products, numpy f64 cross-check
 *   rowwise / g128 quant   exact-rational rounding (fractions.Fraction),
 *                          numpy float16 RNE, pack/unpack bijection
 *   w8a8 accumulators      numpy int64 matmul
 *   attention              closed forms (uniform keys -> mean of v, one
 *                          unmasked key -> that v row, all masked -> NaN),
 *                          numpy f64 softmax / matmul, scale invariance
 *   conversions            numpy astype (f32, f16), exact rationals (bf16),
 *                          closed forms for Rust `as` (saturation, NaN)
 *   e4m3 encode / decode   torch.float8_e4m3fn on all 256 codes and on every
 *                          midpoint / boundary / special value; rowwise FP8
 *                          quantize: exact-rational checks of the scale and
 *                          of |x/s - decode(q)| <= half a step
 *   silu / mlp             closed forms (sigmoid(0)=1/2, limits), math.exp
 */
#ifndef TQ_ORACLE_H
#define TQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QuantDType (crates/theano-quantize/src/qconfig.rs:5-10) */
enum { TQO_INT8 = 0, TQO_UINT8 = 1, TQO_INT4 = 2, TQO_FP8 = 3 };

int tqo_bits(int dtype);
int tqo_is_signed(int dtype);
double tqo_qmin(int dtype);
double tqo_qmax(int dtype);

/* quantize.rs:8-55 */
void tqo_quantize_tensor(const double* x, int64_t n, double scale, double zero_point,
                         int dtype, double* q);
void tqo_dequantize_tensor(const double* q, int64_t n, double scale, double zero_point,
                           double* out);
void tqo_quantize_per_tensor(const double* x, int64_t n, int dtype, double* q,
                             double* scale, double* zero_point);
void tqo_fake_quantize(const double* x, int64_t n, double scale, double zero_point,
                       int dtype, double* out);

/* observer.rs:42-136.  state = {min, max, initialized} */
void tqo_minmax_observe(double* state3, const double* values, int64_t n);
void tqo_minmax_scale_zp(const double* state3, int dtype, double* scale, double* zp);
void tqo_perchannel_observe(double* mins, double* maxs, int64_t channels,
                            const double* values, int64_t n);
void tqo_perchannel_scales_zps(const double* mins, const double* maxs, int64_t channels,
                               int dtype, double* scales, double* zps);
void tqo_perchannel_global_scale_zp(const double* mins, const double* maxs,
                                    int64_t channels, int dtype, double* scale, double* zp);

/* tensor_ops.rs:379-410 (mm, i-p-j order), linear.rs:111-121 (x W^T + b) */
void tqo_mm(const double* a, const double* b, int64_t m, int64_t k, int64_t n, double* c);
void tqo_linear(const double* x, int64_t m, const double* w, const float* bias_or_null,
                int64_t n, int64_t k, double* y);
double tqo_sigmoid(double x);
double tqo_silu_module(double x);

/* conversions used by the build-defined formats (IEEE RNE) */
uint16_t tqo_f64_to_f16_bits(double x);
double tqo_f16_bits_to_f64(uint16_t h);
uint16_t tqo_f32_to_bf16_bits(float x);
double tqo_bf16_bits_to_f64(uint16_t b);

/* build-defined: symmetric per-row INT8 (observer stats + quantize_tensor) */
void tqo_quantize_i8_rowwise(const float* w, int64_t rows, int64_t k, int8_t* q, float* s);
void tqo_dequantize_i8_rowwise(const int8_t* q, const float* s, int64_t rows, int64_t k,
                               float* w_hat);
/* build-defined: symmetric INT4, group 128 along K, two nibbles per byte */
void tqo_quantize_i4_g128(const float* w, int64_t rows, int64_t k, uint8_t* packed,
                          uint16_t* s_f16);
void tqo_dequantize_i4_g128(const uint8_t* packed, const uint16_t* s_f16, int64_t rows,
                            int64_t k, float* w_hat);

/* reference Linear over dequantized weights (f64 result) */
void tqo_linear_w8(const float* x, int64_t m, const int8_t* q, const float* s,
                   const float* bias_or_null, int64_t n, int64_t k, double* y);
void tqo_linear_w4g128_bf16(const uint16_t* x_bf16, int64_t m, const uint8_t* packed,
                            const uint16_t* s_f16, const float* bias_or_null, int64_t n,
                            int64_t k, double* y);
void tqo_linear_w4g128_f32(const float* x, int64_t m, const uint8_t* packed,
                           const uint16_t* s_f16, const float* bias_or_null, int64_t n,
                           int64_t k, double* y);

/* build-defined W8A8 */
void tqo_gemm_w8a8_acc(const int8_t* qa, const int8_t* qw, int64_t m, int64_t n, int64_t k,
                       int32_t* acc);
void tqo_linear_w8a8(const int8_t* qa, const float* sa, const int8_t* qw, const float* sw,
                     const float* bias_or_null, int64_t m, int64_t n, int64_t k, double* y);

/* build-defined FP8 (OCP e4m3, bias 7, max 448, S.1111.111 = NaN), per-row scales */
double tqo_e4m3_to_f64(uint8_t b);
uint8_t tqo_f32_to_e4m3(float x);
void tqo_quantize_fp8_rowwise(const float* w, int64_t rows, int64_t k, uint8_t* q, float* s);
void tqo_dequantize_fp8_rowwise(const uint8_t* q, const float* s, int64_t rows, int64_t k,
                                float* w_hat);
void tqo_linear_fp8(const uint8_t* qa, const float* sa, const uint8_t* qw, const float* sw,
                    const float* bias_or_null, int64_t m, int64_t n, int64_t k, double* y);

/* build-defined element conversion (DType order F16 BF16 F32 F64 U8 I8 I16 I32
 * I64 Bool): dst = cast(f64(src)), RNE for floats, Rust `as` for integers */
uint16_t tqo_f64_to_bf16_bits(double x);
int64_t tqo_dtype_size(int dtype);
void tqo_convert(const void* src, int src_dtype, void* dst, int dst_dtype, int64_t n);

/* attention core of MultiheadAttention::forward_with_mask (transformer.rs:95-142) */
void tqo_attention(const double* q, const double* k, const double* v, const double* mask_or_null,
                   int64_t mask_batch, int64_t B, int64_t S, int64_t H, int64_t D, double* out);

/* build-defined quantized Llama FFN: y = (SiLU(x Wg^T) * (x Wu^T)) Wd^T */
void tqo_mlp_w4g128(const uint16_t* x_bf16, int64_t m, int64_t d, int64_t f,
                    const uint8_t* pg, const uint16_t* sg, const uint8_t* pu,
                    const uint16_t* su, const uint8_t* pd, const uint16_t* sd, double* y);

#ifdef __cplusplus
}
#endif
#endif
