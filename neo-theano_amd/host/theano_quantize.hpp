// theano_quantize.hpp -- C++ host layer of the MI355X quantized-inference path.
//
// Mirrors the Rust-facing API of neo-theano's `theano-quantize` crate
// (crates/theano-quantize/src/lib.rs:9-11) and the Module contract of
// crates/theano-nn/src/module.rs:8-55 over the C ABI of libtq.so (tq.h):
//
//   Rust                                        here
//   Result<T, TheanoError>                      theano::Result<T>, theano::TheanoError
//   Tensor (f64 values + shape)                 theano::Tensor
//   quantize_tensor / dequantize_tensor /       theano::quantize::quantize_tensor / ...
//     quantize_per_tensor / fake_quantize         (same arguments, same f64 results)
//   Observer, MinMaxObserver,                   theano::quantize::Observer, ...
//     PerChannelMinMaxObserver
//   QuantDType, QConfig                         theano::quantize::QuantDType, QConfig
//   Linear::from_tensors(W, b).forward(x)       theano::nn::QuantizedLinear
//
// Host-side functions take and return host data like the crate does (they
// upload, run the GPU kernels on the object's HIP stream and download); the
// *_device members work on device buffers for callers that keep tensors
// resident in HBM.  Errors are returned as Result values where the crate
// returns Result; where the crate cannot fail (dequantize_tensor,
// Module::forward) a failure of the GPU throws TheanoError, the counterpart of
// the crate's panic / unwrap.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <map>
#include <optional>
#include <stdexcept>
#include <string>
#include <tuple>
#include <utility>
#include <variant>
#include <vector>

#include "tq.h"

namespace theano {

// ----------------------------------------------------------------- errors

// TheanoError (crates/theano-types/src/error.rs:7-56).  GPU failures arrive as
// RocmError::KernelError and convert to RuntimeError (theano-rocm/src/error.rs:55-73).
class TheanoError : public std::runtime_error {
   public:
    enum class Kind { InvalidArgument, ShapeMismatch, RuntimeError, OutOfMemory };
    TheanoError(Kind kind, const std::string& msg) : std::runtime_error(msg), kind_(kind) {}
    Kind kind() const { return kind_; }
    static TheanoError invalid_argument(const std::string& m) { return {Kind::InvalidArgument, m}; }
    static TheanoError shape_mismatch(const std::string& m) { return {Kind::ShapeMismatch, m}; }
    static TheanoError runtime(const std::string& m) { return {Kind::RuntimeError, m}; }
    static TheanoError out_of_memory(const std::string& m) { return {Kind::OutOfMemory, m}; }
    // maps a tq_status (+ tq_last_error()) of a failed libtq call
    static TheanoError from_status(int status, const char* what);

   private:
    Kind kind_;
};

// Result<T, TheanoError>
template <class T>
class Result {
   public:
    Result(T value) : v_(std::move(value)) {}
    Result(TheanoError err) : v_(std::move(err)) {}
    bool is_ok() const { return v_.index() == 0; }
    bool is_err() const { return v_.index() == 1; }
    T& unwrap() & {
        if (is_err()) throw std::get<1>(v_);
        return std::get<0>(v_);
    }
    T unwrap() && {
        if (is_err()) throw std::get<1>(v_);
        return std::move(std::get<0>(v_));
    }
    const TheanoError& unwrap_err() const {
        if (is_ok()) throw std::logic_error("unwrap_err on an Ok value");
        return std::get<1>(v_);
    }

   private:
    std::variant<T, TheanoError> v_;
};

template <>
class Result<void> {
   public:
    Result() = default;
    Result(TheanoError err) : e_(std::move(err)) {}
    bool is_ok() const { return !e_.has_value(); }
    bool is_err() const { return e_.has_value(); }
    void unwrap() const {
        if (e_) throw *e_;
    }
    const TheanoError& unwrap_err() const {
        if (!e_) throw std::logic_error("unwrap_err on an Ok value");
        return *e_;
    }

   private:
    std::optional<TheanoError> e_;
};

// ----------------------------------------------------------------- tensors

// Host tensor: f64 values and a shape, the data model of theano-core's Tensor
// (every value is held and handed over as f64, tensor.rs:333-337).
class Tensor {
   public:
    Tensor() = default;
    // Tensor::from_slice (tensor_create.rs:88-90); the element count must match the shape.
    static Tensor from_slice(std::vector<double> data, std::vector<size_t> shape);
    static Tensor zeros(std::vector<size_t> shape);
    static Tensor ones(std::vector<size_t> shape);
    static Tensor scalar(double v) { return from_slice({v}, {}); }

    const std::vector<size_t>& shape() const { return shape_; }
    size_t ndim() const { return shape_.size(); }
    size_t numel() const { return data_.size(); }
    Result<std::vector<double>> to_vec_f64() const { return data_; }
    Result<double> item() const;
    const double* data() const { return data_.data(); }

   private:
    std::vector<double> data_;
    std::vector<size_t> shape_;
};

namespace rocm {

// A device allocation owned by the host layer (the C ABI itself allocates nothing).
template <class T>
class DeviceBuffer {
   public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t n);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_) {
        o.p_ = nullptr;
        o.n_ = 0;
    }
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;

    T* data() { return p_; }
    const T* data() const { return p_; }
    size_t size() const { return n_; }
    // host <-> device copies on `stream` (synchronous with respect to the host)
    void upload(const T* src, size_t n, hipStream_t stream);
    void download(T* dst, size_t n, hipStream_t stream) const;
    std::vector<T> to_host(hipStream_t stream) const;

   private:
    T* p_ = nullptr;
    size_t n_ = 0;
};

}  // namespace rocm

namespace quantize {

// --------------------------------------------------------- dtypes / config

// QuantDType (crates/theano-quantize/src/qconfig.rs:5-41), same order as tq_qdtype.
class QuantDType {
   public:
    enum Kind { Int8_ = TQ_QINT8, UInt8_ = TQ_QUINT8, Int4_ = TQ_QINT4, FP8_ = TQ_QFP8 };
    constexpr QuantDType(Kind k) : k_(k) {}
    static const QuantDType Int8, UInt8, Int4, FP8;
    size_t bits() const;
    bool is_signed() const;
    double qmin() const;
    double qmax() const;
    int abi() const { return static_cast<int>(k_); }
    const char* name() const;
    bool operator==(const QuantDType& o) const { return k_ == o.k_; }
    bool operator!=(const QuantDType& o) const { return k_ != o.k_; }

   private:
    Kind k_;
};
inline const QuantDType QuantDType::Int8{QuantDType::Int8_};
inline const QuantDType QuantDType::UInt8{QuantDType::UInt8_};
inline const QuantDType QuantDType::Int4{QuantDType::Int4_};
inline const QuantDType QuantDType::FP8{QuantDType::FP8_};

// QConfig (qconfig.rs:44-76)
struct QConfig {
    QuantDType weight_dtype = QuantDType::Int8;
    QuantDType activation_dtype = QuantDType::UInt8;
    bool symmetric = true;
    bool per_channel = false;
    static QConfig default_int8() { return {QuantDType::Int8, QuantDType::UInt8, true, false}; }
    static QConfig default_int4() { return {QuantDType::Int4, QuantDType::Int8, true, true}; }
    static QConfig default_() { return default_int8(); }
};

// --------------------------------------------------------- the crate's functions

// quantize_tensor (quantize.rs:8-19): codes as f64, computed in f64 on the GPU.
Result<std::vector<double>> quantize_tensor(const Tensor& tensor, double scale, double zero_point,
                                            QuantDType dtype);
// dequantize_tensor (quantize.rs:22-27)
std::vector<double> dequantize_tensor(const std::vector<double>& quantized, double scale, double zero_point);
// quantize_per_tensor (quantize.rs:30-48): (codes, scale, zero_point)
Result<std::tuple<std::vector<double>, double, double>> quantize_per_tensor(const Tensor& tensor,
                                                                            QuantDType dtype);
// fake_quantize (quantize.rs:51-55): same shape as the input
Result<Tensor> fake_quantize(const Tensor& tensor, double scale, double zero_point, QuantDType dtype);

// Observer (observer.rs:6-10)
class Observer {
   public:
    virtual ~Observer() = default;
    virtual void observe(const std::vector<double>& values) = 0;
    virtual std::pair<double, double> compute_scale_zero_point(QuantDType dtype) const = 0;
    virtual void reset() = 0;
};

// MinMaxObserver (observer.rs:12-73): running min/max held on the device.
class MinMaxObserver : public Observer {
   public:
    MinMaxObserver();
    static MinMaxObserver default_() { return MinMaxObserver(); }
    void observe(const std::vector<double>& values) override;
    std::pair<double, double> compute_scale_zero_point(QuantDType dtype) const override;
    void reset() override;
    double min_val() const;
    double max_val() const;

   private:
    rocm::DeviceBuffer<double> state_;
    bool initialized_ = false;
};

// PerChannelMinMaxObserver (observer.rs:75-136): values laid out [channels, ...].
class PerChannelMinMaxObserver : public Observer {
   public:
    explicit PerChannelMinMaxObserver(size_t num_channels);
    void observe(const std::vector<double>& values) override;
    std::vector<std::pair<double, double>> scales_and_zero_points(QuantDType dtype) const;
    // average of the per-channel (scale, zero_point) (observer.rs:123-129)
    std::pair<double, double> compute_scale_zero_point(QuantDType dtype) const override;
    void reset() override;
    size_t num_channels() const { return channels_; }

   private:
    size_t channels_;
    rocm::DeviceBuffer<double> state_;
};

// --------------------------------------------------------- weight formats

// Symmetric per-output-channel INT8 weight held in HBM: codes int8 [rows, cols],
// scales f32 [rows] (s = f32(max(absmax / 127, 1e-10))).
struct Int8Weight {
    size_t rows = 0, cols = 0;
    rocm::DeviceBuffer<int8_t> codes;
    rocm::DeviceBuffer<float> scales;
};

// Symmetric INT4 with groups of 128 along K held in HBM: packed u8 [rows, cols/2]
// (low nibble = even k), f16 scales [rows, cols/128]; plus the row-tiled copy
// the decode GEMV streams (tile_rows > 0 once made).
struct Int4Weight {
    size_t rows = 0, cols = 0;
    rocm::DeviceBuffer<uint8_t> packed;
    rocm::DeviceBuffer<uint16_t> scales;
    int64_t tile_rows = 0;
    rocm::DeviceBuffer<uint8_t> packed_tiled;
    rocm::DeviceBuffer<uint16_t> scales_tiled;
};

// Symmetric per-output-channel FP8 (OCP e4m3: bias 7, largest finite 448, the
// range of QuantDType::FP8) held in HBM: codes u8 [rows, cols] (e4m3 bit
// patterns), scales f32 [rows] (s = f32(max(absmax / 448, 1e-10))).
struct Fp8Weight {
    size_t rows = 0, cols = 0;
    rocm::DeviceBuffer<uint8_t> codes;
    rocm::DeviceBuffer<float> scales;
};

// The weight's f32 values (f64 host values are rounded to f32 first, the
// element type the device formats are defined on).
Result<Int8Weight> quantize_per_channel_i8(const Tensor& weight, hipStream_t stream = nullptr);
Result<Int4Weight> quantize_i4_g128(const Tensor& weight, hipStream_t stream = nullptr);
Result<Fp8Weight> quantize_per_channel_fp8(const Tensor& weight, hipStream_t stream = nullptr);
Result<Tensor> dequantize(const Int8Weight& w, hipStream_t stream = nullptr);
Result<Tensor> dequantize(const Int4Weight& w, hipStream_t stream = nullptr);
Result<Tensor> dequantize(const Fp8Weight& w, hipStream_t stream = nullptr);
// value of an e4m3 bit pattern (NaN for S.1111.111)
double e4m3_value(uint8_t code);

}  // namespace quantize

namespace serialize {
class SafeTensorsFile;  // theano_serialize.hpp
}

namespace nn {

// Module (crates/theano-nn/src/module.rs:8-55) over host tensors: the quantized
// inference path has no autograd, so Tensor stands where the crate has Variable.
class Module {
   public:
    virtual ~Module() = default;
    virtual Tensor forward(const Tensor& input) const = 0;
    virtual std::vector<Tensor> parameters() const = 0;
    virtual std::vector<std::pair<std::string, Tensor>> named_parameters() const;
    virtual size_t num_parameters() const;
    std::map<std::string, Tensor> state_dict() const;
};

// y = x . dequant(W)^T + b: Linear::from_tensors(dequantize(W), b).forward(x)
// (crates/theano-nn/src/linear.rs:65-75, 111-121) with W quantized in HBM.
// Mode from the QConfig:
//   weight Int8, activations not Int8 -> "w8":   INT8 weight-only, f32 activations
//   weight Int8, activations Int8     -> "w8a8": per-row dynamic INT8 activations
//   weight Int4                       -> "w4":   INT4 g128 weight-only, bf16 activations
//   weight FP8, activations FP8       -> "fp8":  FP8 e4m3 weights, per-row dynamic FP8 activations
//   weight FP8, activations not FP8   -> "fp8_weight": FP8 e4m3 weight-only, f32 activations
class QuantizedLinear : public Module {
   public:
    enum class Mode { W8, W8A8, W4, FP8, FP8Weight };
    static Result<QuantizedLinear> from_tensors(const Tensor& weight, const std::optional<Tensor>& bias,
                                                const quantize::QConfig& qconfig = quantize::QConfig::default_int8(),
                                                hipStream_t stream = nullptr);

    // x [M, in] or [in]; returns [M, out] or [out] (f64 values of the f32 result)
    Tensor forward(const Tensor& input) const override;
    Result<Tensor> try_forward(const Tensor& input) const;
    // Device-resident forward: x is f32 [m, in] (w8, w8a8, fp8) or bf16 bits [m, in]
    // (w4), y is f32 [m, out]; enqueued on `stream`, no host synchronisation.  w8a8
    // and fp8 need `act_codes` (one byte per element, [m, in]) and `act_scales`
    // (f32 [m]) device scratch.  With m <= kFusedA8MaxM both quantize x inside the
    // decode GEMV (tq_gemv_w8a8 / tq_gemv_fp8a8) when K % 16 == 0, K <= 8192 and x
    // is 16-byte aligned, otherwise fp8 runs the GEMV on the fake-quantized
    // activations held in `workspace` (workspace_bytes(m) bytes); larger m
    // quantize x into the scratch and run the GEMM (its skinny kernel up to 16
    // tokens: faster than the fused GEMV from 3 tokens).  w4 runs the
    // tiled GEMV in passes of 16 tokens up to m = kTiledPassesMaxM (at N = 14336,
    // K = 4096: 19 us at m = 17-32 against 21-24 us for the prefill GEMM on its
    // 64-row tiles, 37 against 25.5 us at m = 64), the prefill GEMM beyond, with `workspace`
    // (workspace_bytes(m) bytes) when given.
    Result<void> forward_device(const void* x, int64_t m, float* y, hipStream_t stream,
                                int8_t* act_codes = nullptr, float* act_scales = nullptr,
                                void* workspace = nullptr, size_t workspace_bytes = 0) const;
    static constexpr int64_t kTiledPassesMaxM = 32;
    static constexpr int64_t kFusedA8MaxM = 2;
    // device scratch for m tokens: the w4 prefill path and the fp8 GEMV on
    // fake-quantized activations (m <= kFusedA8MaxM); 0 otherwise
    size_t workspace_bytes(int64_t m) const;
    // Quantized checkpoint entries under `name` (layout in theano_serialize.hpp):
    // codes and scales as stored on the device, loaded back without re-quantizing.
    Result<void> save(serialize::SafeTensorsFile& file, const std::string& name) const;
    static Result<QuantizedLinear> load(const serialize::SafeTensorsFile& file, const std::string& name,
                                        hipStream_t stream = nullptr);

    std::vector<Tensor> parameters() const override;
    std::vector<std::pair<std::string, Tensor>> named_parameters() const override;
    size_t num_parameters() const override;
    size_t in_features() const { return in_; }
    size_t out_features() const { return out_; }
    Mode mode() const { return mode_; }
    hipStream_t stream() const { return stream_; }

   private:
    Mode mode_ = Mode::W8;
    size_t in_ = 0, out_ = 0;
    hipStream_t stream_ = nullptr;
    quantize::Int8Weight w8_;
    quantize::Int4Weight w4_;
    quantize::Fp8Weight fp8_;
    std::optional<rocm::DeviceBuffer<float>> bias_;
};

// Llama-style FFN on INT4 g128 weights: y = (SiLU(x Wg^T) * (x Wu^T)) Wd^T
// (Linear + SiLU (activation.rs:66-79) + Tensor::mul), bf16 activations, the
// SiLU(gate) * up intermediate in f32.
class QuantizedMLP : public Module {
   public:
    static Result<QuantizedMLP> from_tensors(const Tensor& gate, const Tensor& up, const Tensor& down,
                                             hipStream_t stream = nullptr);
    Tensor forward(const Tensor& input) const override;
    Result<Tensor> try_forward(const Tensor& input) const;
    // device bytes of intermediates for m tokens (tq_mlp_w4g128_decode_workspace_bytes
    // on the decode path, tq_mlp_w4g128_workspace_bytes otherwise)
    size_t workspace_bytes(int64_t m) const;
    // x bf16 bits [m, d], workspace of workspace_bytes(m) bytes, y f32 [m, d]
    Result<void> forward_device(const uint16_t* x, int64_t m, void* workspace, size_t workspace_bytes, float* y,
                                hipStream_t stream) const;
    std::vector<Tensor> parameters() const override;
    size_t num_parameters() const override { return 3 * d_ * f_; }
    // Quantized checkpoint entries under `name` (layout in theano_serialize.hpp)
    Result<void> save(serialize::SafeTensorsFile& file, const std::string& name) const;
    static Result<QuantizedMLP> load(const serialize::SafeTensorsFile& file, const std::string& name,
                                     hipStream_t stream = nullptr);
    size_t hidden() const { return d_; }
    size_t intermediate() const { return f_; }
    // decode shapes (D and F at most 16384; 1 <= m <= 8, or m <= kDecodeMaxM where
    // D <= kDecodeOnePassD, whose gate/up takes 16 tokens in one launch) run
    // tq_mlp_w4g128_decode on row-tiled copies of the weights, in passes of
    // kDecodePassM tokens; others tq_mlp_w4g128 (at D = 4096, F = 14336: 35-48 us
    // for 5-16 tokens and 66-78 us for 17-24, 93 us at 32, against 85-88 us for
    // the prefill FFN on its 64-row tiles)
    static constexpr int64_t kDecodeMaxM = 28;
    static constexpr int64_t kDecodePassM = 16;
    static constexpr size_t kDecodeOnePassD = 4096;
    bool decode_path(int64_t m) const {
        return gu_tiled_.size() > 0 && m >= 1 && (m <= 8 || (m <= kDecodeMaxM && d_ <= kDecodeOnePassD));
    }

   private:
    void make_decode_copies();
    size_t d_ = 0, f_ = 0;
    hipStream_t stream_ = nullptr;
    quantize::Int4Weight gate_, up_, down_;
    rocm::DeviceBuffer<uint8_t> gu_tiled_;  // gate and up interleaved in 64-row tiles
    rocm::DeviceBuffer<uint16_t> gu_scales_tiled_;
};

// f32 -> bf16 bits, round to nearest even (NaN stays NaN)
uint16_t f32_to_bf16(float x);
float bf16_to_f32(uint16_t b);

// MultiheadAttention (crates/theano-nn/src/transformer.rs:9-162) with its q/k/v
// and out projections as QuantizedLinear consumers.  q, k and v are quantized
// row by row, so their concatenation [3E, E] has exactly the three codes: the
// module holds one fused q/k/v QuantizedLinear (one GEMM / GEMV for
// self-attention) and the out projection; the attention core (scores, additive
// mask, softmax, P V) is tq_attention_f32 on the f32 projections.  Inputs and
// outputs are [batch, seq, E].  Cross-attention (distinct query / key / value)
// runs the fused projection on each input and keeps its third.
class QuantizedMultiheadAttention : public Module {
   public:
    static Result<QuantizedMultiheadAttention> from_tensors(
        size_t num_heads, const Tensor& wq, const Tensor& wk, const Tensor& wv, const Tensor& wo,
        const std::optional<Tensor>& bq = std::nullopt, const std::optional<Tensor>& bk = std::nullopt,
        const std::optional<Tensor>& bv = std::nullopt, const std::optional<Tensor>& bo = std::nullopt,
        const quantize::QConfig& qconfig = quantize::QConfig::default_int8(), hipStream_t stream = nullptr);

    // self-attention (Module::forward, transformer.rs:145-150)
    Tensor forward(const Tensor& input) const override;
    // transformer.rs:86-142; mask additive [batch or 1, (1,) seq, seq]
    Result<Tensor> forward_with_mask(const Tensor& query, const Tensor& key, const Tensor& value,
                                     const std::optional<Tensor>& mask) const;
    Tensor forward_qkv(const Tensor& query, const Tensor& key, const Tensor& value) const;

    std::vector<Tensor> parameters() const override;
    // q_proj.*, k_proj.*, v_proj.*, out_proj.* (weight, weight_scale, bias)
    std::vector<std::pair<std::string, Tensor>> named_parameters() const override;
    size_t num_parameters() const override;
    size_t embed_dim() const { return e_; }
    size_t num_heads() const { return h_; }
    size_t head_dim() const { return e_ / h_; }
    const QuantizedLinear& qkv() const { return qkv_; }
    const QuantizedLinear& out_proj() const { return out_; }

   private:
    size_t e_ = 0, h_ = 1;
    hipStream_t stream_ = nullptr;
    QuantizedLinear qkv_, out_;
};

}  // namespace nn
}  // namespace theano
