// bench_storage.cpp -- measurements of the device storage layer, printed as one
// JSON object (bench.py runs this as a child process):
//   * from_host_f64: host f64 values -> device BF16 / F32 storage (pinned
//     double-buffered H2D of the f64 payload + tq_convert), GB/s of f64 input;
//   * to_host_f64 of an F32 storage (D2H + host widening), GB/s of f64 output;
//   * allocate + free of a cached block vs hipMalloc + hipFree, microseconds;
//   * one decode-sized QuantizedLinear (INT4 g128, 4096 -> 14336, M = 1) through
//     the host Tensor API (upload, GEMV, download per call) vs the
//     device-resident forward (activations stay in HBM), microseconds per call.
#include <hip/hip_runtime.h>

#include <chrono>
#include <cstdio>
#include <random>
#include <vector>

#include "theano_quantize.hpp"
#include "theano_rocm.hpp"

using namespace theano;
using clk = std::chrono::steady_clock;

namespace {

double seconds_since(clk::time_point t0) { return std::chrono::duration<double>(clk::now() - t0).count(); }

std::vector<double> randn(size_t n, double std, uint64_t seed) {
    std::mt19937_64 g(seed);
    std::normal_distribution<double> d(0.0, std);
    std::vector<double> v(n);
    for (auto& x : v) x = d(g);
    return v;
}

}  // namespace

int main() {
    auto dev = rocm::DeviceManager::global().get_device(0).unwrap();
    const size_t n = size_t(64) << 20;  // 64 Mi values = 512 MB of f64
    const std::vector<double> host = randn(n, 1.0, 1);
    std::printf("{");

    // H2D + convert
    for (DType dt : {DType::BF16, DType::F32}) {
        (void)rocm::RocmStorage::from_host_f64(dev, host.data(), n, dt).unwrap();  // warm the pool and staging
        const int reps = 3;
        auto t0 = clk::now();
        for (int i = 0; i < reps; ++i) {
            auto s = rocm::RocmStorage::from_host_f64(dev, host.data(), n, dt).unwrap();
            (void)dev->synchronize();
        }
        const double gbs = 8.0 * n * reps / seconds_since(t0) / 1e9;
        std::printf("\"from_host_f64_to_%s_GB/s\": %.2f, ", dtype_name(dt), gbs);
    }
    {
        auto s = rocm::RocmStorage::from_host_f64(dev, host.data(), n, DType::F32).unwrap();
        (void)s.to_host_f64().unwrap();
        auto t0 = clk::now();
        const int reps = 3;
        for (int i = 0; i < reps; ++i) (void)s.to_host_f64().unwrap();
        std::printf("\"to_host_f64_from_float32_GB/s\": %.2f, ", 8.0 * n * reps / seconds_since(t0) / 1e9);
    }

    // allocator vs driver
    {
        const size_t bytes = size_t(8) << 20;
        auto& a = dev->allocator();
        a.free(a.allocate(bytes).unwrap());
        const int reps = 2000;
        auto t0 = clk::now();
        for (int i = 0; i < reps; ++i) a.free(a.allocate(bytes).unwrap());
        const double cached_us = seconds_since(t0) / reps * 1e6;
        void* p = nullptr;
        (void)hipMalloc(&p, bytes);
        (void)hipFree(p);
        const int dreps = 200;
        t0 = clk::now();
        for (int i = 0; i < dreps; ++i) {
            (void)hipMalloc(&p, bytes);
            (void)hipFree(p);
        }
        const double driver_us = seconds_since(t0) / dreps * 1e6;
        std::printf("\"alloc_free_8MiB_cached_us\": %.3f, \"alloc_free_8MiB_hipMalloc_us\": %.3f, ", cached_us, driver_us);
    }

    // decode Linear: host API vs device-resident
    {
        const size_t k = 4096, out = 14336;
        const auto layer = nn::QuantizedLinear::from_tensors(Tensor::from_slice(randn(out * k, 0.02, 2), {out, k}),
                                                             std::nullopt, quantize::QConfig::default_int4())
                               .unwrap();
        const Tensor x = Tensor::from_slice(randn(k, 1.0, 3), {1, k});
        const DeviceTensor xd = DeviceTensor::from_host(x, dev, DType::BF16).unwrap();
        (void)layer.forward(x);
        (void)nn::forward(layer, xd).unwrap();
        (void)dev->synchronize();
        const int reps = 200;
        auto t0 = clk::now();
        for (int i = 0; i < reps; ++i) (void)layer.forward(x);
        const double host_us = seconds_since(t0) / reps * 1e6;
        t0 = clk::now();
        for (int i = 0; i < reps; ++i) (void)nn::forward(layer, xd).unwrap();
        (void)dev->synchronize();
        const double dev_us = seconds_since(t0) / reps * 1e6;
        std::printf("\"linear_w4_m1_host_api_us\": %.2f, \"linear_w4_m1_device_resident_us\": %.2f, ", host_us, dev_us);
    }
    const auto st = dev->allocator().stats();
    std::printf("\"allocator_mallocs\": %zu, \"allocator_cache_hits\": %zu}\n", st.num_mallocs, st.num_cache_hits);
    return 0;
}
