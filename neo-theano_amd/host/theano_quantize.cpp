// theano_quantize.cpp -- C++ host layer over libtq.so (see theano_quantize.hpp).
#include "theano_quantize.hpp"
#include "theano_serialize.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <numeric>

namespace theano {

namespace {

// Throws the TheanoError of a failed libtq call (a GPU failure has no
// Result to go into in the crate's infallible signatures either).
void check(int status, const char* what) {
    if (status != TQ_OK) throw TheanoError::from_status(status, what);
}

void check_hip(hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory) throw TheanoError::out_of_memory(std::string(what) + ": out of device memory");
    if (e != hipSuccess) throw TheanoError::runtime(std::string("HIP kernel launch error: ") + what + ": " +
                                                    hipGetErrorString(e));
}

size_t shape_numel(const std::vector<size_t>& shape) {
    return std::accumulate(shape.begin(), shape.end(), size_t{1}, [](size_t a, size_t b) { return a * b; });
}

std::string shape_str(const std::vector<size_t>& shape) {
    std::string s = "[";
    for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
    return s + "]";
}

// Runs `f` and turns a thrown TheanoError into an Err.
template <class T, class F>
Result<T> capture(F&& f) {
    try {
        return f();
    } catch (const TheanoError& e) {
        return e;
    }
}

}  // namespace

TheanoError TheanoError::from_status(int status, const char* what) {
    const std::string msg = std::string(what) + ": " + tq_last_error();
    switch (status) {
        case TQ_EINVAL:
            return invalid_argument(msg);
        case TQ_ENOMEM:
            return out_of_memory(msg);
        default:
            return runtime("HIP kernel launch error: " + msg);
    }
}

// ----------------------------------------------------------------- Tensor

Tensor Tensor::from_slice(std::vector<double> data, std::vector<size_t> shape) {
    if (shape_numel(shape) != data.size())
        throw TheanoError::shape_mismatch("Tensor::from_slice: " + std::to_string(data.size()) +
                                          " values for shape " + shape_str(shape));
    Tensor t;
    t.data_ = std::move(data);
    t.shape_ = std::move(shape);
    return t;
}

Tensor Tensor::zeros(std::vector<size_t> shape) {
    std::vector<double> d(shape_numel(shape), 0.0);
    return from_slice(std::move(d), std::move(shape));
}

Tensor Tensor::ones(std::vector<size_t> shape) {
    std::vector<double> d(shape_numel(shape), 1.0);
    return from_slice(std::move(d), std::move(shape));
}

Result<double> Tensor::item() const {
    if (data_.size() != 1)
        return TheanoError::invalid_argument("item(): tensor has " + std::to_string(data_.size()) + " elements");
    return data_[0];
}

// ----------------------------------------------------------------- DeviceBuffer

namespace rocm {

template <class T>
DeviceBuffer<T>::DeviceBuffer(size_t n) : n_(n) {
    if (n) check_hip(hipMalloc(reinterpret_cast<void**>(&p_), n * sizeof(T)), "hipMalloc");
}

template <class T>
DeviceBuffer<T>::~DeviceBuffer() {
    if (p_) (void)hipFree(p_);
}

template <class T>
DeviceBuffer<T>& DeviceBuffer<T>::operator=(DeviceBuffer&& o) noexcept {
    if (this != &o) {
        if (p_) (void)hipFree(p_);
        p_ = o.p_;
        n_ = o.n_;
        o.p_ = nullptr;
        o.n_ = 0;
    }
    return *this;
}

template <class T>
void DeviceBuffer<T>::upload(const T* src, size_t n, hipStream_t stream) {
    if (n > n_) throw TheanoError::invalid_argument("DeviceBuffer::upload: too many elements");
    if (!n) return;
    check_hip(hipMemcpyAsync(p_, src, n * sizeof(T), hipMemcpyHostToDevice, stream), "upload");
    check_hip(hipStreamSynchronize(stream), "upload");
}

template <class T>
void DeviceBuffer<T>::download(T* dst, size_t n, hipStream_t stream) const {
    if (n > n_) throw TheanoError::invalid_argument("DeviceBuffer::download: too many elements");
    if (!n) return;
    check_hip(hipMemcpyAsync(dst, p_, n * sizeof(T), hipMemcpyDeviceToHost, stream), "download");
    check_hip(hipStreamSynchronize(stream), "download");
}

template <class T>
std::vector<T> DeviceBuffer<T>::to_host(hipStream_t stream) const {
    std::vector<T> v(n_);
    download(v.data(), n_, stream);
    return v;
}

template class DeviceBuffer<double>;
template class DeviceBuffer<float>;
template class DeviceBuffer<int8_t>;
template class DeviceBuffer<uint8_t>;
template class DeviceBuffer<uint16_t>;
template class DeviceBuffer<int32_t>;

}  // namespace rocm

using rocm::DeviceBuffer;

namespace quantize {

// ----------------------------------------------------------------- QuantDType

namespace {
struct DTypeInfo {
    int bits, is_signed;
    double qmin, qmax;
};
DTypeInfo info(int q) {
    DTypeInfo d{};
    check(tq_qdtype_info(q, &d.bits, &d.is_signed, &d.qmin, &d.qmax), "QuantDType");
    return d;
}
}  // namespace

size_t QuantDType::bits() const { return static_cast<size_t>(info(abi()).bits); }
bool QuantDType::is_signed() const { return info(abi()).is_signed != 0; }
double QuantDType::qmin() const { return info(abi()).qmin; }
double QuantDType::qmax() const { return info(abi()).qmax; }
const char* QuantDType::name() const {
    switch (k_) {
        case Int8_:
            return "Int8";
        case UInt8_:
            return "UInt8";
        case Int4_:
            return "Int4";
        default:
            return "FP8";
    }
}

// ----------------------------------------------------------------- primitives

Result<std::vector<double>> quantize_tensor(const Tensor& tensor, double scale, double zero_point,
                                            QuantDType dtype) {
    return capture<std::vector<double>>([&]() -> Result<std::vector<double>> {
        const size_t n = tensor.numel();
        DeviceBuffer<double> x(n), q(n);
        x.upload(tensor.data(), n, nullptr);
        const int st = tq_quantize_tensor_f64(x.data(), static_cast<int64_t>(n), scale, zero_point, dtype.abi(),
                                              q.data(), nullptr);
        if (st != TQ_OK) return TheanoError::from_status(st, "quantize_tensor");
        return q.to_host(nullptr);
    });
}

std::vector<double> dequantize_tensor(const std::vector<double>& quantized, double scale, double zero_point) {
    const size_t n = quantized.size();
    DeviceBuffer<double> q(n), out(n);
    q.upload(quantized.data(), n, nullptr);
    check(tq_dequantize_tensor_f64(q.data(), static_cast<int64_t>(n), scale, zero_point, out.data(), nullptr),
          "dequantize_tensor");
    return out.to_host(nullptr);
}

Result<std::tuple<std::vector<double>, double, double>> quantize_per_tensor(const Tensor& tensor,
                                                                            QuantDType dtype) {
    using R = std::tuple<std::vector<double>, double, double>;
    return capture<R>([&]() -> Result<R> {
        const size_t n = tensor.numel();
        DeviceBuffer<double> x(n), q(n), szp(2);
        DeviceBuffer<uint8_t> ws(TQ_PER_TENSOR_WORKSPACE);
        x.upload(tensor.data(), n, nullptr);
        const int st = tq_quantize_per_tensor_f64(x.data(), static_cast<int64_t>(n), dtype.abi(), q.data(),
                                                  szp.data(), ws.data(), nullptr);
        if (st != TQ_OK) return TheanoError::from_status(st, "quantize_per_tensor");
        const std::vector<double> sz = szp.to_host(nullptr);
        return R{q.to_host(nullptr), sz[0], sz[1]};
    });
}

Result<Tensor> fake_quantize(const Tensor& tensor, double scale, double zero_point, QuantDType dtype) {
    return capture<Tensor>([&]() -> Result<Tensor> {
        const size_t n = tensor.numel();
        DeviceBuffer<double> x(n), out(n);
        x.upload(tensor.data(), n, nullptr);
        const int st = tq_fake_quantize_f64(x.data(), static_cast<int64_t>(n), scale, zero_point, dtype.abi(),
                                            out.data(), nullptr);
        if (st != TQ_OK) return TheanoError::from_status(st, "fake_quantize");
        return Tensor::from_slice(out.to_host(nullptr), tensor.shape());
    });
}

// ----------------------------------------------------------------- observers

namespace {
std::pair<double, double> scale_zp(double mn, double mx, bool initialized, QuantDType dtype) {
    double s = 0, z = 0;
    check(tq_observer_scale_zp(mn, mx, initialized ? 1 : 0, dtype.abi(), &s, &z), "compute_scale_zero_point");
    return {s, z};
}
}  // namespace

MinMaxObserver::MinMaxObserver() : state_(2) { reset(); }

void MinMaxObserver::observe(const std::vector<double>& values) {
    DeviceBuffer<double> x(values.size());
    x.upload(values.data(), values.size(), nullptr);
    check(tq_minmax_observe_f64(x.data(), static_cast<int64_t>(values.size()), state_.data(), nullptr),
          "MinMaxObserver::observe");
    check_hip(hipStreamSynchronize(nullptr), "MinMaxObserver::observe");
    initialized_ = true;
}

double MinMaxObserver::min_val() const { return state_.to_host(nullptr)[0]; }
double MinMaxObserver::max_val() const { return state_.to_host(nullptr)[1]; }

std::pair<double, double> MinMaxObserver::compute_scale_zero_point(QuantDType dtype) const {
    const std::vector<double> st = state_.to_host(nullptr);
    return scale_zp(st[0], st[1], initialized_, dtype);
}

void MinMaxObserver::reset() {
    check(tq_minmax_reset_f64(state_.data(), 1, nullptr), "MinMaxObserver::reset");
    initialized_ = false;
}

PerChannelMinMaxObserver::PerChannelMinMaxObserver(size_t num_channels)
    : channels_(num_channels), state_(2 * num_channels) {
    if (num_channels == 0) throw TheanoError::invalid_argument("PerChannelMinMaxObserver: zero channels");
    reset();
}

void PerChannelMinMaxObserver::observe(const std::vector<double>& values) {
    DeviceBuffer<double> x(values.size());
    x.upload(values.data(), values.size(), nullptr);
    check(tq_minmax_observe_per_channel_f64(x.data(), static_cast<int64_t>(values.size()),
                                            static_cast<int64_t>(channels_), state_.data(), nullptr),
          "PerChannelMinMaxObserver::observe");
    check_hip(hipStreamSynchronize(nullptr), "PerChannelMinMaxObserver::observe");
}

std::vector<std::pair<double, double>> PerChannelMinMaxObserver::scales_and_zero_points(QuantDType dtype) const {
    const std::vector<double> st = state_.to_host(nullptr);
    std::vector<std::pair<double, double>> out;
    out.reserve(channels_);
    // observer.rs:93-106 has no `initialized` check
    for (size_t c = 0; c < channels_; ++c) out.push_back(scale_zp(st[2 * c], st[2 * c + 1], true, dtype));
    return out;
}

std::pair<double, double> PerChannelMinMaxObserver::compute_scale_zero_point(QuantDType dtype) const {
    const auto sz = scales_and_zero_points(dtype);
    double s = 0, z = 0;
    for (const auto& p : sz) s += p.first;
    for (const auto& p : sz) z += p.second;
    return {s / static_cast<double>(sz.size()), z / static_cast<double>(sz.size())};
}

void PerChannelMinMaxObserver::reset() {
    check(tq_minmax_reset_f64(state_.data(), static_cast<int64_t>(channels_), nullptr),
          "PerChannelMinMaxObserver::reset");
}

// ----------------------------------------------------------------- weight formats

namespace {

// [rows, cols] view of a 2-D tensor's values rounded to f32
std::vector<float> as_f32_matrix(const Tensor& w, const char* what, size_t* rows, size_t* cols) {
    if (w.ndim() != 2)
        throw TheanoError::invalid_argument(std::string(what) + ": weight must be 2-D, got " + shape_str(w.shape()));
    *rows = w.shape()[0];
    *cols = w.shape()[1];
    std::vector<float> f(w.numel());
    for (size_t i = 0; i < f.size(); ++i) f[i] = static_cast<float>(w.data()[i]);
    return f;
}

Tensor to_tensor(const std::vector<float>& v, std::vector<size_t> shape) {
    return Tensor::from_slice(std::vector<double>(v.begin(), v.end()), std::move(shape));
}

}  // namespace

Result<Int8Weight> quantize_per_channel_i8(const Tensor& weight, hipStream_t stream) {
    return capture<Int8Weight>([&]() -> Result<Int8Weight> {
        Int8Weight w;
        const std::vector<float> f = as_f32_matrix(weight, "quantize_per_channel_i8", &w.rows, &w.cols);
        DeviceBuffer<float> src(f.size());
        src.upload(f.data(), f.size(), stream);
        w.codes = DeviceBuffer<int8_t>(w.rows * w.cols);
        w.scales = DeviceBuffer<float>(w.rows);
        const int st = tq_quantize_i8_rowwise(src.data(), static_cast<int64_t>(w.rows), static_cast<int64_t>(w.cols),
                                              w.codes.data(), w.scales.data(),
                                              reinterpret_cast<tq_stream_t>(stream));
        if (st != TQ_OK) return TheanoError::from_status(st, "quantize_per_channel_i8");
        check_hip(hipStreamSynchronize(stream), "quantize_per_channel_i8");
        return std::move(w);
    });
}

Result<Fp8Weight> quantize_per_channel_fp8(const Tensor& weight, hipStream_t stream) {
    return capture<Fp8Weight>([&]() -> Result<Fp8Weight> {
        Fp8Weight w;
        const std::vector<float> f = as_f32_matrix(weight, "quantize_per_channel_fp8", &w.rows, &w.cols);
        DeviceBuffer<float> src(f.size());
        src.upload(f.data(), f.size(), stream);
        w.codes = DeviceBuffer<uint8_t>(w.rows * w.cols);
        w.scales = DeviceBuffer<float>(w.rows);
        const int st = tq_quantize_fp8_rowwise(src.data(), static_cast<int64_t>(w.rows),
                                               static_cast<int64_t>(w.cols), w.codes.data(), w.scales.data(),
                                               reinterpret_cast<tq_stream_t>(stream));
        if (st != TQ_OK) return TheanoError::from_status(st, "quantize_per_channel_fp8");
        check_hip(hipStreamSynchronize(stream), "quantize_per_channel_fp8");
        return std::move(w);
    });
}

double e4m3_value(uint8_t code) {
    const double sign = (code & 0x80) ? -1.0 : 1.0;
    const int e = (code >> 3) & 0xF, m = code & 7;
    if (e == 15 && m == 7) return std::nan("");
    return e == 0 ? sign * std::ldexp(m, -9) : sign * std::ldexp(8 + m, e - 10);
}

// Row-tiled copy of w for the decode GEMV; tile_rows 0 picks tq_w4g128_tile_rows(rows).
void make_tiled(Int4Weight& w, hipStream_t stream, int64_t tile_rows = 0);

Result<Int4Weight> quantize_i4_g128(const Tensor& weight, hipStream_t stream) {
    return capture<Int4Weight>([&]() -> Result<Int4Weight> {
        Int4Weight w;
        const std::vector<float> f = as_f32_matrix(weight, "quantize_i4_g128", &w.rows, &w.cols);
        if (w.cols % 128 != 0)
            return TheanoError::invalid_argument("quantize_i4_g128: K=" + std::to_string(w.cols) +
                                                 " is not a multiple of the group size 128");
        DeviceBuffer<float> src(f.size());
        src.upload(f.data(), f.size(), stream);
        w.packed = DeviceBuffer<uint8_t>(w.rows * w.cols / 2);
        w.scales = DeviceBuffer<uint16_t>(w.rows * w.cols / 128);
        const auto ts = reinterpret_cast<tq_stream_t>(stream);
        int st = tq_quantize_i4_g128(src.data(), static_cast<int64_t>(w.rows), static_cast<int64_t>(w.cols),
                                     w.packed.data(), w.scales.data(), ts);
        if (st != TQ_OK) return TheanoError::from_status(st, "quantize_i4_g128");
        make_tiled(w, stream);
        check_hip(hipStreamSynchronize(stream), "quantize_i4_g128");
        return std::move(w);
    });
}

void make_tiled(Int4Weight& w, hipStream_t stream, int64_t tile_rows) {
    if (w.cols > 16384 || w.rows == 0) return;
    // row-tiled copy for the decode GEMV (a permutation of the packed bytes)
    const int64_t t = tile_rows > 0 ? tile_rows : tq_w4g128_tile_rows(static_cast<int64_t>(w.rows));
    if (t <= 0) throw TheanoError::runtime("tiled INT4 copy: tile size query failed");
    const size_t padded = (w.rows + t - 1) / t * t;
    w.packed_tiled = DeviceBuffer<uint8_t>(padded * w.cols / 2);
    w.scales_tiled = DeviceBuffer<uint16_t>(padded * w.cols / 128);
    check(tq_repack_w4g128_tiled(w.packed.data(), w.scales.data(), static_cast<int64_t>(w.rows),
                                 static_cast<int64_t>(w.cols), t, w.packed_tiled.data(), w.scales_tiled.data(),
                                 reinterpret_cast<tq_stream_t>(stream)),
          "tiled INT4 copy");
    w.tile_rows = t;
}

Result<Tensor> dequantize(const Int8Weight& w, hipStream_t stream) {
    return capture<Tensor>([&]() -> Result<Tensor> {
        DeviceBuffer<float> out(w.rows * w.cols);
        const int st = tq_dequantize_i8_rowwise(w.codes.data(), w.scales.data(), static_cast<int64_t>(w.rows),
                                                static_cast<int64_t>(w.cols), out.data(),
                                                reinterpret_cast<tq_stream_t>(stream));
        if (st != TQ_OK) return TheanoError::from_status(st, "dequantize");
        return to_tensor(out.to_host(stream), {w.rows, w.cols});
    });
}

Result<Tensor> dequantize(const Fp8Weight& w, hipStream_t stream) {
    return capture<Tensor>([&]() -> Result<Tensor> {
        DeviceBuffer<float> out(w.rows * w.cols);
        const int st = tq_dequantize_fp8_rowwise(w.codes.data(), w.scales.data(), static_cast<int64_t>(w.rows),
                                                 static_cast<int64_t>(w.cols), out.data(),
                                                 reinterpret_cast<tq_stream_t>(stream));
        if (st != TQ_OK) return TheanoError::from_status(st, "dequantize");
        return to_tensor(out.to_host(stream), {w.rows, w.cols});
    });
}

Result<Tensor> dequantize(const Int4Weight& w, hipStream_t stream) {
    return capture<Tensor>([&]() -> Result<Tensor> {
        DeviceBuffer<float> out(w.rows * w.cols);
        const int st = tq_dequantize_i4_g128(w.packed.data(), w.scales.data(), static_cast<int64_t>(w.rows),
                                             static_cast<int64_t>(w.cols), out.data(),
                                             reinterpret_cast<tq_stream_t>(stream));
        if (st != TQ_OK) return TheanoError::from_status(st, "dequantize");
        return to_tensor(out.to_host(stream), {w.rows, w.cols});
    });
}

}  // namespace quantize

// ----------------------------------------------------------------- nn

namespace nn {

using quantize::Int4Weight;
using quantize::Int8Weight;
using quantize::QConfig;
using quantize::QuantDType;

uint16_t f32_to_bf16(float x) {
    uint32_t b;
    std::memcpy(&b, &x, 4);
    if ((b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu)) return static_cast<uint16_t>((b >> 16) | 0x40);
    b += 0x7FFFu + ((b >> 16) & 1u);  // round to nearest even
    return static_cast<uint16_t>(b >> 16);
}

float bf16_to_f32(uint16_t h) {
    const uint32_t b = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

std::vector<std::pair<std::string, Tensor>> Module::named_parameters() const {
    std::vector<std::pair<std::string, Tensor>> out;
    const auto ps = parameters();
    for (size_t i = 0; i < ps.size(); ++i) out.emplace_back("param_" + std::to_string(i), ps[i]);
    return out;
}

size_t Module::num_parameters() const {
    size_t n = 0;
    for (const auto& p : parameters()) n += p.numel();
    return n;
}

std::map<std::string, Tensor> Module::state_dict() const {
    std::map<std::string, Tensor> out;
    for (auto& kv : named_parameters()) out.emplace(kv.first, kv.second);
    return out;
}

namespace {

// rows x cols activations of a 1-D or 2-D input; `squeeze` when 1-D
std::vector<double> input_rows(const Tensor& x, size_t in, const char* what, size_t* m, bool* squeeze) {
    if (x.ndim() == 1 && x.shape()[0] == in) {
        *m = 1;
        *squeeze = true;
    } else if (x.ndim() == 2 && x.shape()[1] == in) {
        *m = x.shape()[0];
        *squeeze = false;
    } else {
        throw TheanoError::shape_mismatch(std::string(what) + ": expected [*, " + std::to_string(in) + "], got " +
                                          shape_str(x.shape()));
    }
    return std::vector<double>(x.data(), x.data() + x.numel());
}

Tensor output_tensor(const std::vector<float>& y, size_t m, size_t n, bool squeeze) {
    std::vector<double> d(y.begin(), y.end());
    return squeeze ? Tensor::from_slice(std::move(d), {n}) : Tensor::from_slice(std::move(d), {m, n});
}

std::vector<uint16_t> to_bf16(const std::vector<double>& v) {
    std::vector<uint16_t> out(v.size());
    for (size_t i = 0; i < v.size(); ++i) out[i] = f32_to_bf16(static_cast<float>(v[i]));
    return out;
}

}  // namespace

namespace {
// shapes the fused-activation decode GEMVs take
bool fused_a8_ok(const void* x, const void* q, int64_t k) {
    return k > 0 && k <= 8192 && k % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(q) % 16 == 0;
}
}  // namespace

Result<QuantizedLinear> QuantizedLinear::from_tensors(const Tensor& weight, const std::optional<Tensor>& bias,
                                                      const QConfig& qconfig, hipStream_t stream) {
    return capture<QuantizedLinear>([&]() -> Result<QuantizedLinear> {
        QuantizedLinear l;
        l.stream_ = stream;
        if (qconfig.weight_dtype == QuantDType::Int4) {
            l.mode_ = Mode::W4;
            auto r = quantize::quantize_i4_g128(weight, stream);
            if (r.is_err()) return r.unwrap_err();
            l.w4_ = std::move(r).unwrap();
            l.out_ = l.w4_.rows;
            l.in_ = l.w4_.cols;
        } else if (qconfig.weight_dtype == QuantDType::Int8) {
            l.mode_ = qconfig.activation_dtype == QuantDType::Int8 ? Mode::W8A8 : Mode::W8;
            auto r = quantize::quantize_per_channel_i8(weight, stream);
            if (r.is_err()) return r.unwrap_err();
            l.w8_ = std::move(r).unwrap();
            l.out_ = l.w8_.rows;
            l.in_ = l.w8_.cols;
        } else if (qconfig.weight_dtype == QuantDType::FP8) {
            l.mode_ = qconfig.activation_dtype == QuantDType::FP8 ? Mode::FP8 : Mode::FP8Weight;
            auto r = quantize::quantize_per_channel_fp8(weight, stream);
            if (r.is_err()) return r.unwrap_err();
            l.fp8_ = std::move(r).unwrap();
            l.out_ = l.fp8_.rows;
            l.in_ = l.fp8_.cols;
        } else {
            return TheanoError::invalid_argument(std::string("QuantizedLinear: unsupported weight dtype ") +
                                                 qconfig.weight_dtype.name());
        }
        if (bias) {
            if (bias->numel() != l.out_)
                return TheanoError::shape_mismatch("QuantizedLinear: bias " + shape_str(bias->shape()) +
                                                   " for " + std::to_string(l.out_) + " outputs");
            std::vector<float> b(l.out_);
            for (size_t i = 0; i < l.out_; ++i) b[i] = static_cast<float>(bias->data()[i]);
            l.bias_.emplace(l.out_);
            l.bias_->upload(b.data(), b.size(), stream);
        }
        return std::move(l);
    });
}

size_t QuantizedLinear::workspace_bytes(int64_t m) const {
    if (mode_ == Mode::FP8 && m <= kFusedA8MaxM) return static_cast<size_t>(m) * in_ * sizeof(float);
    if (mode_ != Mode::W4 || m <= 16 || (w4_.tile_rows > 0 && m <= kTiledPassesMaxM)) return 0;
    return static_cast<size_t>(tq_gemm_w4g128_bf16_workspace_bytes(m, static_cast<int64_t>(in_)));
}

Result<void> QuantizedLinear::forward_device(const void* x, int64_t m, float* y, hipStream_t stream, int8_t* act_codes,
                                             float* act_scales, void* workspace, size_t workspace_bytes) const {
    const auto ts = reinterpret_cast<tq_stream_t>(stream);
    const float* b = bias_ ? bias_->data() : nullptr;
    const int64_t n = static_cast<int64_t>(out_), k = static_cast<int64_t>(in_);
    int st = TQ_OK;
    switch (mode_) {
        case Mode::W4: {
            const auto* xb = static_cast<const uint16_t*>(x);
            if (m <= kTiledPassesMaxM && w4_.tile_rows > 0) {
                for (int64_t m0 = 0; m0 < m && st == TQ_OK; m0 += 16) {
                    const int64_t mm = std::min<int64_t>(16, m - m0);
                    st = tq_gemv_w4g128_tiled(xb + m0 * k, mm, w4_.packed_tiled.data(), w4_.scales_tiled.data(), b,
                                              n, k, w4_.tile_rows, y + m0 * n, ts);
                }
            } else if (m <= 16)
                st = tq_gemv_w4g128(xb, m, w4_.packed.data(), w4_.scales.data(), b, n, k, y, ts);
            else if (workspace)
                st = tq_gemm_w4g128_bf16_ws(xb, m, w4_.packed.data(), w4_.scales.data(), b, n, k, workspace,
                                            static_cast<int64_t>(workspace_bytes), y, ts);
            else
                st = tq_gemm_w4g128_bf16(xb, m, w4_.packed.data(), w4_.scales.data(), b, n, k, y, ts);
            break;
        }
        case Mode::W8: {
            const auto* xf = static_cast<const float*>(x);
            for (int64_t m0 = 0; m0 < m && st == TQ_OK; m0 += 16) {
                const int64_t mm = std::min<int64_t>(16, m - m0);
                st = tq_gemv_w8(xf + m0 * k, mm, w8_.codes.data(), w8_.scales.data(), b, n, k, y + m0 * n, ts);
            }
            break;
        }
        case Mode::W8A8: {
            // quantize-in-GEMV (one launch) for 1-2 tokens; beyond, quantize + the
            // GEMM's skinny kernel is faster (4096 x 4096: 10.6 against 12.0 us at
            // m = 3, 12.5 against 52.3 us at m = 16)
            if (m <= kFusedA8MaxM && fused_a8_ok(x, w8_.codes.data(), k)) {
                st = tq_gemv_w8a8(static_cast<const float*>(x), m, w8_.codes.data(), w8_.scales.data(), b, n, k, y,
                                  ts);
                break;
            }
            if (!act_codes || !act_scales)
                return TheanoError::invalid_argument("QuantizedLinear::forward_device: w8a8 needs activation scratch");
            st = tq_quantize_i8_rowwise(static_cast<const float*>(x), m, k, act_codes, act_scales, ts);
            if (st == TQ_OK)
                st = tq_gemm_w8a8(act_codes, act_scales, w8_.codes.data(), w8_.scales.data(), b, m, n, k, nullptr, y,
                                  ts);
            break;
        }
        case Mode::FP8: {  // as W8A8 (FP8 at 4096 x 4096: 10.0 against 12.9 us at m = 3)
            if (m <= kFusedA8MaxM && fused_a8_ok(x, fp8_.codes.data(), k)) {
                st = tq_gemv_fp8a8(static_cast<const float*>(x), m, fp8_.codes.data(), fp8_.scales.data(), b, n, k,
                                   y, ts);
                break;
            }
            if (!act_codes || !act_scales)
                return TheanoError::invalid_argument("QuantizedLinear::forward_device: fp8 needs activation scratch");
            auto* qa = reinterpret_cast<uint8_t*>(act_codes);
            if (m > kFusedA8MaxM) {
                st = tq_quantize_fp8_rowwise(static_cast<const float*>(x), m, k, qa, act_scales, ts);
                if (st == TQ_OK)
                    st = tq_gemm_fp8(qa, act_scales, fp8_.codes.data(), fp8_.scales.data(), b, m, n, k, y, ts);
                break;
            }
            // decode: the GEMV over x_hat = e4m3(qa) * sa, the GEMM's activation values
            if (!workspace || workspace_bytes < this->workspace_bytes(m))
                return TheanoError::invalid_argument(
                    "QuantizedLinear::forward_device: fp8 with m <= 2 needs workspace_bytes(m) of workspace");
            auto* xq = static_cast<float*>(workspace);
            st = tq_fake_quantize_fp8_rowwise(static_cast<const float*>(x), m, k, qa, act_scales, xq, ts);
            if (st == TQ_OK) st = tq_gemv_fp8(xq, m, fp8_.codes.data(), fp8_.scales.data(), b, n, k, y, ts);
            break;
        }
        case Mode::FP8Weight: {
            const auto* xf = static_cast<const float*>(x);
            for (int64_t m0 = 0; m0 < m && st == TQ_OK; m0 += 16) {
                const int64_t mm = std::min<int64_t>(16, m - m0);
                st = tq_gemv_fp8(xf + m0 * k, mm, fp8_.codes.data(), fp8_.scales.data(), b, n, k, y + m0 * n, ts);
            }
            break;
        }
    }
    if (st != TQ_OK) return TheanoError::from_status(st, "QuantizedLinear::forward");
    return {};
}

Result<Tensor> QuantizedLinear::try_forward(const Tensor& input) const {
    return capture<Tensor>([&]() -> Result<Tensor> {
        size_t m = 0;
        bool squeeze = false;
        const std::vector<double> xv = input_rows(input, in_, "QuantizedLinear::forward", &m, &squeeze);
        DeviceBuffer<float> y(m * out_);
        Result<void> r;
        if (mode_ == Mode::W4) {
            const std::vector<uint16_t> xb = to_bf16(xv);
            DeviceBuffer<uint16_t> xd(xb.size());
            xd.upload(xb.data(), xb.size(), stream_);
            const size_t wsb = workspace_bytes(static_cast<int64_t>(m));
            DeviceBuffer<uint8_t> ws(std::max<size_t>(wsb, 1));
            r = forward_device(xd.data(), static_cast<int64_t>(m), y.data(), stream_, nullptr, nullptr,
                               wsb ? ws.data() : nullptr, wsb);
        } else {
            const std::vector<float> xf(xv.begin(), xv.end());
            DeviceBuffer<float> xd(xf.size());
            xd.upload(xf.data(), xf.size(), stream_);
            if (mode_ == Mode::W8A8 || mode_ == Mode::FP8) {
                DeviceBuffer<int8_t> qa(m * in_);
                DeviceBuffer<float> sa(m);
                const size_t wsb = workspace_bytes(static_cast<int64_t>(m));
                DeviceBuffer<uint8_t> ws(std::max<size_t>(wsb, 1));
                r = forward_device(xd.data(), static_cast<int64_t>(m), y.data(), stream_, qa.data(), sa.data(),
                                   wsb ? ws.data() : nullptr, wsb);
                if (r.is_ok()) check_hip(hipStreamSynchronize(stream_), "QuantizedLinear::forward");
            } else {
                r = forward_device(xd.data(), static_cast<int64_t>(m), y.data(), stream_);
            }
        }
        if (r.is_err()) return r.unwrap_err();
        return output_tensor(y.to_host(stream_), m, out_, squeeze);
    });
}

Tensor QuantizedLinear::forward(const Tensor& input) const { return try_forward(input).unwrap(); }

std::vector<std::pair<std::string, Tensor>> QuantizedLinear::named_parameters() const {
    // codes and scales as f64 tensors, like the crate's f64 parameter data
    std::vector<std::pair<std::string, Tensor>> out;
    if (mode_ == Mode::W4) {
        const auto p = w4_.packed.to_host(stream_);
        const auto s = w4_.scales.to_host(stream_);
        std::vector<double> codes(out_ * in_), sc(s.size());
        for (size_t i = 0; i < p.size(); ++i) {
            codes[2 * i] = static_cast<double>(static_cast<int8_t>(static_cast<uint8_t>(p[i] << 4)) >> 4);
            codes[2 * i + 1] = static_cast<double>(static_cast<int8_t>(p[i]) >> 4);
        }
        for (size_t i = 0; i < s.size(); ++i) {
            // f16 bits -> value
            const uint16_t h = s[i];
            const int e = (h >> 10) & 0x1F, f = h & 0x3FF;
            const double mag = e ? std::ldexp(1.0 + f / 1024.0, e - 15) : std::ldexp(f / 1024.0, -14);
            sc[i] = (h & 0x8000) ? -mag : mag;
        }
        out.emplace_back("weight", Tensor::from_slice(std::move(codes), {out_, in_}));
        out.emplace_back("weight_scale", Tensor::from_slice(std::move(sc), {out_, in_ / 128}));
    } else if (mode_ == Mode::FP8 || mode_ == Mode::FP8Weight) {
        const auto q = fp8_.codes.to_host(stream_);
        const auto s = fp8_.scales.to_host(stream_);
        std::vector<double> codes(q.size());
        for (size_t i = 0; i < q.size(); ++i) codes[i] = quantize::e4m3_value(q[i]);
        out.emplace_back("weight", Tensor::from_slice(std::move(codes), {out_, in_}));
        out.emplace_back("weight_scale", Tensor::from_slice(std::vector<double>(s.begin(), s.end()), {out_}));
    } else {
        const auto q = w8_.codes.to_host(stream_);
        const auto s = w8_.scales.to_host(stream_);
        out.emplace_back("weight", Tensor::from_slice(std::vector<double>(q.begin(), q.end()), {out_, in_}));
        out.emplace_back("weight_scale", Tensor::from_slice(std::vector<double>(s.begin(), s.end()), {out_}));
    }
    if (bias_) {
        const auto b = bias_->to_host(stream_);
        out.emplace_back("bias", Tensor::from_slice(std::vector<double>(b.begin(), b.end()), {out_}));
    }
    return out;
}

std::vector<Tensor> QuantizedLinear::parameters() const {
    std::vector<Tensor> out;
    for (auto& kv : named_parameters()) out.push_back(kv.second);
    return out;
}

size_t QuantizedLinear::num_parameters() const { return in_ * out_ + (bias_ ? out_ : 0); }

Result<QuantizedMLP> QuantizedMLP::from_tensors(const Tensor& gate, const Tensor& up, const Tensor& down,
                                                hipStream_t stream) {
    return capture<QuantizedMLP>([&]() -> Result<QuantizedMLP> {
        if (gate.ndim() != 2 || up.shape() != gate.shape() || down.ndim() != 2 || down.shape()[0] != gate.shape()[1] ||
            down.shape()[1] != gate.shape()[0])
            return TheanoError::shape_mismatch("QuantizedMLP: gate/up must be [F, D] and down [D, F]");
        QuantizedMLP mlp;
        mlp.stream_ = stream;
        mlp.f_ = gate.shape()[0];
        mlp.d_ = gate.shape()[1];
        for (auto [src, dst] : {std::pair{&gate, &mlp.gate_}, std::pair{&up, &mlp.up_}, std::pair{&down, &mlp.down_}}) {
            auto r = quantize::quantize_i4_g128(*src, stream);
            if (r.is_err()) return r.unwrap_err();
            *dst = std::move(r).unwrap();
        }
        mlp.make_decode_copies();
        return std::move(mlp);
    });
}

void QuantizedMLP::make_decode_copies() {
    // down keeps the tiled copy every INT4 weight gets; gate and up run from one
    // interleaved copy instead of their own
    gate_.packed_tiled = DeviceBuffer<uint8_t>();
    gate_.scales_tiled = DeviceBuffer<uint16_t>();
    gate_.tile_rows = 0;
    up_.packed_tiled = DeviceBuffer<uint8_t>();
    up_.scales_tiled = DeviceBuffer<uint16_t>();
    up_.tile_rows = 0;
    if (d_ == 0 || f_ == 0 || d_ > 16384 || f_ > 16384 || down_.tile_rows == 0) return;
    // down in 32-row tiles: two K halves per tile give 2 D / 32 blocks, one
    // round on 256 CUs at D = 4096
    if (down_.tile_rows != 32) quantize::make_tiled(down_, stream_, 32);
    const size_t tiles = (f_ + 31) / 32;
    gu_tiled_ = DeviceBuffer<uint8_t>(tiles * 64 * d_ / 2);
    gu_scales_tiled_ = DeviceBuffer<uint16_t>(tiles * 64 * d_ / 128);
    check(tq_repack_w4g128_gate_up_tiled(gate_.packed.data(), gate_.scales.data(), up_.packed.data(),
                                         up_.scales.data(), static_cast<int64_t>(f_), static_cast<int64_t>(d_),
                                         gu_tiled_.data(), gu_scales_tiled_.data(),
                                         reinterpret_cast<tq_stream_t>(stream_)),
          "QuantizedMLP: tiled gate/up copy");
    check_hip(hipStreamSynchronize(stream_), "QuantizedMLP: tiled gate/up copy");
}

size_t QuantizedMLP::workspace_bytes(int64_t m) const {
    if (decode_path(m))
        return static_cast<size_t>(tq_mlp_w4g128_decode_workspace_bytes(
            std::min<int64_t>(m, kDecodePassM), static_cast<int64_t>(d_), static_cast<int64_t>(f_)));
    return static_cast<size_t>(
        tq_mlp_w4g128_workspace_bytes(m, static_cast<int64_t>(d_), static_cast<int64_t>(f_)));
}

Result<void> QuantizedMLP::forward_device(const uint16_t* x, int64_t m, void* workspace, size_t workspace_bytes,
                                          float* y, hipStream_t stream) const {
    if (decode_path(m)) {
        const int64_t d = static_cast<int64_t>(d_);
        // passes of kDecodePassM tokens, ordered on the stream, share the workspace
        for (int64_t m0 = 0; m0 < m; m0 += kDecodePassM) {
            const int64_t mm = std::min<int64_t>(kDecodePassM, m - m0);
            const int st = tq_mlp_w4g128_decode(x + m0 * d, mm, d, static_cast<int64_t>(f_), gu_tiled_.data(),
                                                gu_scales_tiled_.data(), down_.packed_tiled.data(),
                                                down_.scales_tiled.data(), down_.tile_rows, workspace,
                                                static_cast<int64_t>(workspace_bytes), y + m0 * d,
                                                reinterpret_cast<tq_stream_t>(stream));
            if (st != TQ_OK) return TheanoError::from_status(st, "QuantizedMLP::forward");
        }
        return {};
    }
    const int st = tq_mlp_w4g128(x, m, static_cast<int64_t>(d_), static_cast<int64_t>(f_), gate_.packed.data(),
                                 gate_.scales.data(), up_.packed.data(), up_.scales.data(), down_.packed.data(),
                                 down_.scales.data(), workspace, static_cast<int64_t>(workspace_bytes), y,
                                 reinterpret_cast<tq_stream_t>(stream));
    if (st != TQ_OK) return TheanoError::from_status(st, "QuantizedMLP::forward");
    return {};
}

Result<Tensor> QuantizedMLP::try_forward(const Tensor& input) const {
    return capture<Tensor>([&]() -> Result<Tensor> {
        size_t m = 0;
        bool squeeze = false;
        const std::vector<double> xv = input_rows(input, d_, "QuantizedMLP::forward", &m, &squeeze);
        const std::vector<uint16_t> xb = to_bf16(xv);
        DeviceBuffer<uint16_t> xd(xb.size());
        xd.upload(xb.data(), xb.size(), stream_);
        DeviceBuffer<uint8_t> ws(std::max<size_t>(workspace_bytes(static_cast<int64_t>(m)), 1));
        DeviceBuffer<float> y(m * d_);
        auto r = forward_device(xd.data(), static_cast<int64_t>(m), ws.data(), ws.size(), y.data(), stream_);
        if (r.is_err()) return r.unwrap_err();
        return output_tensor(y.to_host(stream_), m, d_, squeeze);
    });
}

Tensor QuantizedMLP::forward(const Tensor& input) const { return try_forward(input).unwrap(); }

std::vector<Tensor> QuantizedMLP::parameters() const {
    std::vector<Tensor> out;
    for (const Int4Weight* w : {&gate_, &up_, &down_}) {
        auto t = quantize::dequantize(*w, stream_);
        out.push_back(std::move(t).unwrap());
    }
    return out;
}

// ------------------------------------------------- QuantizedMultiheadAttention

namespace {

// rows [r0, r0 + n) of a [rows, ...] tensor
Tensor row_slice(const Tensor& t, size_t r0, size_t n) {
    const size_t cols = t.ndim() == 2 ? t.shape()[1] : 1;
    std::vector<double> v(t.data() + r0 * cols, t.data() + (r0 + n) * cols);
    return t.ndim() == 2 ? Tensor::from_slice(std::move(v), {n, cols}) : Tensor::from_slice(std::move(v), {n});
}

// y [m, n] f32 = layer(x [m, in] f32) on the device, with the mode's activation
// type and scratch (device buffers owned here, released after the stream syncs)
void run_projection(const QuantizedLinear& l, const float* x, int64_t m, float* y, hipStream_t st) {
    const auto ts = reinterpret_cast<tq_stream_t>(st);
    const size_t k = l.in_features();
    DeviceBuffer<uint16_t> xb;
    const void* xin = x;
    if (l.mode() == QuantizedLinear::Mode::W4) {
        xb = DeviceBuffer<uint16_t>(static_cast<size_t>(m) * k);
        check(tq_convert(x, TQ_DT_F32, xb.data(), TQ_DT_BF16, m * static_cast<int64_t>(k), ts), "bf16 activations");
        xin = xb.data();
    }
    DeviceBuffer<int8_t> codes(static_cast<size_t>(m) * k);
    DeviceBuffer<float> scales(static_cast<size_t>(m));
    const size_t wsb = l.workspace_bytes(m);
    DeviceBuffer<uint8_t> ws(std::max<size_t>(wsb, 1));
    l.forward_device(xin, m, y, st, codes.data(), scales.data(), wsb ? ws.data() : nullptr, wsb).unwrap();
    check_hip(hipStreamSynchronize(st), "QuantizedMultiheadAttention projection");
}

}  // namespace

Result<QuantizedMultiheadAttention> QuantizedMultiheadAttention::from_tensors(
    size_t num_heads, const Tensor& wq, const Tensor& wk, const Tensor& wv, const Tensor& wo,
    const std::optional<Tensor>& bq, const std::optional<Tensor>& bk, const std::optional<Tensor>& bv,
    const std::optional<Tensor>& bo, const QConfig& qconfig, hipStream_t stream) {
    return capture<QuantizedMultiheadAttention>([&]() -> Result<QuantizedMultiheadAttention> {
        if (wq.ndim() != 2 || wq.shape()[0] != wq.shape()[1] || wk.shape() != wq.shape() || wv.shape() != wq.shape() ||
            wo.shape() != wq.shape())
            return TheanoError::shape_mismatch("QuantizedMultiheadAttention: the four weights must be [E, E]");
        const size_t e = wq.shape()[0];
        if (num_heads == 0 || e % num_heads)
            return TheanoError::invalid_argument("QuantizedMultiheadAttention: embed_dim % num_heads != 0");
        std::vector<double> cat;
        cat.reserve(3 * e * e);
        for (const Tensor* w : {&wq, &wk, &wv}) cat.insert(cat.end(), w->data(), w->data() + e * e);
        std::optional<Tensor> bcat;
        if (bq || bk || bv) {
            std::vector<double> b(3 * e, 0.0);
            const std::optional<Tensor>* bs[3] = {&bq, &bk, &bv};
            for (size_t i = 0; i < 3; ++i)
                if (*bs[i]) {
                    if ((*bs[i])->numel() != e)
                        return TheanoError::shape_mismatch("QuantizedMultiheadAttention: bias must be [E]");
                    std::copy((*bs[i])->data(), (*bs[i])->data() + e, b.begin() + i * e);
                }
            bcat = Tensor::from_slice(std::move(b), {3 * e});
        }
        QuantizedMultiheadAttention a;
        a.e_ = e;
        a.h_ = num_heads;
        a.stream_ = stream;
        auto qkv = QuantizedLinear::from_tensors(Tensor::from_slice(std::move(cat), {3 * e, e}), bcat, qconfig, stream);
        if (qkv.is_err()) return qkv.unwrap_err();
        auto out = QuantizedLinear::from_tensors(wo, bo, qconfig, stream);
        if (out.is_err()) return out.unwrap_err();
        a.qkv_ = std::move(qkv).unwrap();
        a.out_ = std::move(out).unwrap();
        return std::move(a);
    });
}

Result<Tensor> QuantizedMultiheadAttention::forward_with_mask(const Tensor& query, const Tensor& key,
                                                              const Tensor& value,
                                                              const std::optional<Tensor>& mask) const {
    return capture<Tensor>([&]() -> Result<Tensor> {
        const auto& sh = query.shape();
        if (query.ndim() != 3 || sh[2] != e_ || key.shape() != sh || value.shape() != sh)
            return TheanoError::shape_mismatch("QuantizedMultiheadAttention: query, key, value must be [batch, seq, " +
                                               std::to_string(e_) + "], got " + shape_str(sh));
        const size_t b = sh[0], s = sh[1], m = b * s;
        int64_t mb = 0;
        if (mask) {
            const auto& ms = mask->shape();
            const bool ok3 = ms.size() == 3 && ms[1] == s && ms[2] == s;
            const bool ok4 = ms.size() == 4 && ms[1] == 1 && ms[2] == s && ms[3] == s;
            if (!(ok3 || ok4) || (ms[0] != 1 && ms[0] != b))
                return TheanoError::shape_mismatch("QuantizedMultiheadAttention: mask must be [batch or 1, (1,) seq, seq]");
            mb = static_cast<int64_t>(ms[0]);
        }
        const hipStream_t st = stream_;
        const bool self = &query == &key && &key == &value;
        // fused projections: [m, 3E] per distinct input
        std::vector<DeviceBuffer<float>> proj;
        for (const Tensor* in : self ? std::vector<const Tensor*>{&query} : std::vector<const Tensor*>{&query, &key, &value}) {
            std::vector<float> xf(in->data(), in->data() + m * e_);
            DeviceBuffer<float> xd(xf.size());
            xd.upload(xf.data(), xf.size(), st);
            proj.emplace_back(m * 3 * e_);
            run_projection(qkv_, xd.data(), static_cast<int64_t>(m), proj.back().data(), st);
        }
        const float* qp = proj[0].data();
        const float* kp = (self ? proj[0].data() : proj[1].data()) + e_;
        const float* vp = (self ? proj[0].data() : proj[2].data()) + 2 * e_;
        DeviceBuffer<float> md;
        if (mask) {
            std::vector<float> mf(mask->data(), mask->data() + mask->numel());
            md = DeviceBuffer<float>(mf.size());
            md.upload(mf.data(), mf.size(), st);
        }
        DeviceBuffer<float> att(m * e_), y(m * e_);
        const int64_t ld = static_cast<int64_t>(3 * e_);
        check(tq_attention_f32(qp, ld, kp, ld, vp, ld, mask ? md.data() : nullptr, mb, static_cast<int64_t>(b),
                               static_cast<int64_t>(s), static_cast<int64_t>(h_), static_cast<int64_t>(e_ / h_),
                               att.data(), static_cast<int64_t>(e_), reinterpret_cast<tq_stream_t>(st)),
              "QuantizedMultiheadAttention attention");
        run_projection(out_, att.data(), static_cast<int64_t>(m), y.data(), st);
        const auto yv = y.to_host(st);
        return Tensor::from_slice(std::vector<double>(yv.begin(), yv.end()), sh);
    });
}

Tensor QuantizedMultiheadAttention::forward(const Tensor& input) const {
    return forward_with_mask(input, input, input, std::nullopt).unwrap();
}

Tensor QuantizedMultiheadAttention::forward_qkv(const Tensor& query, const Tensor& key, const Tensor& value) const {
    return forward_with_mask(query, key, value, std::nullopt).unwrap();
}

std::vector<std::pair<std::string, Tensor>> QuantizedMultiheadAttention::named_parameters() const {
    std::vector<std::pair<std::string, Tensor>> out;
    const auto fused = qkv_.named_parameters();
    const char* names[3] = {"q_proj", "k_proj", "v_proj"};
    for (size_t i = 0; i < 3; ++i)
        for (const auto& kv : fused) out.emplace_back(std::string(names[i]) + "." + kv.first, row_slice(kv.second, i * e_, e_));
    for (const auto& kv : out_.named_parameters()) out.emplace_back("out_proj." + kv.first, kv.second);
    return out;
}

std::vector<Tensor> QuantizedMultiheadAttention::parameters() const {
    std::vector<Tensor> out;
    for (auto& kv : named_parameters()) out.push_back(kv.second);
    return out;
}

size_t QuantizedMultiheadAttention::num_parameters() const { return qkv_.num_parameters() + out_.num_parameters(); }

}  // namespace nn
}  // namespace theano

// ------------------------------------------------------ quantized checkpoints
namespace theano {
namespace nn {
namespace {

using serialize::SafeTensorsFile;

std::string meta(const SafeTensorsFile& f, const std::string& key) {
    const auto it = f.metadata.find(key);
    if (it == f.metadata.end()) throw TheanoError::runtime("checkpoint: missing metadata '" + key + "'");
    return it->second;
}

size_t meta_size(const SafeTensorsFile& f, const std::string& key) {
    const std::string v = meta(f, key);
    try {
        return static_cast<size_t>(std::stoull(v));
    } catch (...) {
        throw TheanoError::runtime("checkpoint: metadata '" + key + "' is not a size: " + v);
    }
}

template <class T>
std::vector<uint8_t> bytes_of(const DeviceBuffer<T>& b, hipStream_t stream) {
    const std::vector<T> h = b.to_host(stream);
    std::vector<uint8_t> out(h.size() * sizeof(T));
    std::memcpy(out.data(), h.data(), out.size());
    return out;
}

template <class T>
DeviceBuffer<T> device_of(const std::vector<uint8_t>& raw, hipStream_t stream) {
    DeviceBuffer<T> b(raw.size() / sizeof(T));
    b.upload(reinterpret_cast<const T*>(raw.data()), raw.size() / sizeof(T), stream);
    return b;
}

template <class T>
std::vector<uint8_t> get(const SafeTensorsFile& f, const std::string& name, const char* dtype,
                         std::vector<size_t> shape) {
    auto r = f.get_raw(name, dtype, shape);
    if (r.is_err()) throw r.unwrap_err();
    return std::move(r).unwrap();
}

void put(SafeTensorsFile& f, const std::string& name, const char* dtype, std::vector<size_t> shape,
         const std::vector<uint8_t>& raw) {
    auto r = f.add_raw(name, dtype, std::move(shape), raw.data(), raw.size());
    if (r.is_err()) throw r.unwrap_err();
}

void put_int4(SafeTensorsFile& f, const std::string& name, const Int4Weight& w, hipStream_t stream) {
    put(f, name + ".weight", "U8", {w.rows, w.cols / 2}, bytes_of(w.packed, stream));
    put(f, name + ".weight_scale", "F16", {w.rows, w.cols / 128}, bytes_of(w.scales, stream));
}

Int4Weight get_int4(const SafeTensorsFile& f, const std::string& name, size_t rows, size_t cols,
                    hipStream_t stream) {
    if (cols % 128 != 0) throw TheanoError::runtime("checkpoint: '" + name + "' K is not a multiple of 128");
    Int4Weight w;
    w.rows = rows;
    w.cols = cols;
    w.packed = device_of<uint8_t>(get<uint8_t>(f, name + ".weight", "U8", {rows, cols / 2}), stream);
    w.scales = device_of<uint16_t>(get<uint16_t>(f, name + ".weight_scale", "F16", {rows, cols / 128}), stream);
    quantize::make_tiled(w, stream);
    check_hip(hipStreamSynchronize(stream), "checkpoint");
    return w;
}

}  // namespace

Result<void> QuantizedLinear::save(SafeTensorsFile& f, const std::string& name) const {
    return capture<void>([&]() -> Result<void> {
        f.metadata["format"] = serialize::kFormat;
        f.metadata[name + ".in_features"] = std::to_string(in_);
        f.metadata[name + ".out_features"] = std::to_string(out_);
        if (mode_ == Mode::W4) {
            f.metadata[name + ".quant"] = "int4_g128";
            f.metadata[name + ".group_size"] = "128";
            put_int4(f, name, w4_, stream_);
        } else if (mode_ == Mode::FP8 || mode_ == Mode::FP8Weight) {
            f.metadata[name + ".quant"] = mode_ == Mode::FP8 ? "fp8_e4m3_per_channel_a8" : "fp8_e4m3_per_channel";
            put(f, name + ".weight", "F8_E4M3", {out_, in_}, bytes_of(fp8_.codes, stream_));
            put(f, name + ".weight_scale", "F32", {out_}, bytes_of(fp8_.scales, stream_));
        } else {
            f.metadata[name + ".quant"] = mode_ == Mode::W8 ? "int8_per_channel" : "int8_per_channel_a8";
            put(f, name + ".weight", "I8", {out_, in_}, bytes_of(w8_.codes, stream_));
            put(f, name + ".weight_scale", "F32", {out_}, bytes_of(w8_.scales, stream_));
        }
        if (bias_) put(f, name + ".bias", "F32", {out_}, bytes_of(*bias_, stream_));
        return {};
    });
}

Result<QuantizedLinear> QuantizedLinear::load(const SafeTensorsFile& f, const std::string& name,
                                              hipStream_t stream) {
    return capture<QuantizedLinear>([&]() -> Result<QuantizedLinear> {
        if (meta(f, "format") != serialize::kFormat)
            return TheanoError::runtime("checkpoint: format is not " + std::string(serialize::kFormat));
        QuantizedLinear l;
        l.stream_ = stream;
        l.in_ = meta_size(f, name + ".in_features");
        l.out_ = meta_size(f, name + ".out_features");
        const std::string q = meta(f, name + ".quant");
        if (q == "int4_g128") {
            if (meta(f, name + ".group_size") != "128")
                return TheanoError::runtime("checkpoint: '" + name + "' group size is not 128");
            l.mode_ = Mode::W4;
            l.w4_ = get_int4(f, name, l.out_, l.in_, stream);
        } else if (q == "int8_per_channel" || q == "int8_per_channel_a8") {
            l.mode_ = q == "int8_per_channel" ? Mode::W8 : Mode::W8A8;
            l.w8_.rows = l.out_;
            l.w8_.cols = l.in_;
            l.w8_.codes = device_of<int8_t>(get<int8_t>(f, name + ".weight", "I8", {l.out_, l.in_}), stream);
            l.w8_.scales = device_of<float>(get<float>(f, name + ".weight_scale", "F32", {l.out_}), stream);
        } else if (q == "fp8_e4m3_per_channel" || q == "fp8_e4m3_per_channel_a8") {
            l.mode_ = q == "fp8_e4m3_per_channel" ? Mode::FP8Weight : Mode::FP8;
            l.fp8_.rows = l.out_;
            l.fp8_.cols = l.in_;
            l.fp8_.codes = device_of<uint8_t>(get<uint8_t>(f, name + ".weight", "F8_E4M3", {l.out_, l.in_}), stream);
            l.fp8_.scales = device_of<float>(get<float>(f, name + ".weight_scale", "F32", {l.out_}), stream);
        } else {
            return TheanoError::runtime("checkpoint: '" + name + "' has unknown scheme " + q);
        }
        if (f.tensors.count(name + ".bias"))
            l.bias_.emplace(device_of<float>(get<float>(f, name + ".bias", "F32", {l.out_}), stream));
        return std::move(l);
    });
}

Result<void> QuantizedMLP::save(SafeTensorsFile& f, const std::string& name) const {
    return capture<void>([&]() -> Result<void> {
        f.metadata["format"] = serialize::kFormat;
        f.metadata[name + ".quant"] = "mlp_int4_g128";
        f.metadata[name + ".group_size"] = "128";
        f.metadata[name + ".hidden"] = std::to_string(d_);
        f.metadata[name + ".intermediate"] = std::to_string(f_);
        put_int4(f, name + ".gate", gate_, stream_);
        put_int4(f, name + ".up", up_, stream_);
        put_int4(f, name + ".down", down_, stream_);
        return {};
    });
}

Result<QuantizedMLP> QuantizedMLP::load(const SafeTensorsFile& f, const std::string& name, hipStream_t stream) {
    return capture<QuantizedMLP>([&]() -> Result<QuantizedMLP> {
        if (meta(f, "format") != serialize::kFormat)
            return TheanoError::runtime("checkpoint: format is not " + std::string(serialize::kFormat));
        if (meta(f, name + ".quant") != "mlp_int4_g128")
            return TheanoError::runtime("checkpoint: '" + name + "' is not an INT4 MLP");
        QuantizedMLP m;
        m.stream_ = stream;
        m.d_ = meta_size(f, name + ".hidden");
        m.f_ = meta_size(f, name + ".intermediate");
        m.gate_ = get_int4(f, name + ".gate", m.f_, m.d_, stream);
        m.up_ = get_int4(f, name + ".up", m.f_, m.d_, stream);
        m.down_ = get_int4(f, name + ".down", m.d_, m.f_, stream);
        m.make_decode_copies();
        return std::move(m);
    });
}

}  // namespace nn
}  // namespace theano
