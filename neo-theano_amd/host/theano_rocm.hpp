// theano_rocm.hpp -- device storage under the quantized path: the caching
// allocator, device handle and storage of neo-theano's `theano-rocm` crate on
// real HIP memory, and a device-resident tensor for the quantized modules.
//
//   Rust (theano-rocm, theano-core)               here
//   CachingAllocator, Block, AllocatorStats       theano::rocm::CachingAllocator, Block, AllocatorStats
//     (crates/theano-rocm/src/allocator.rs:29-305)
//   RocmDevice, DeviceProperties, DeviceManager   theano::rocm::RocmDevice, DeviceProperties, DeviceManager
//     (crates/theano-rocm/src/device.rs:10-213)
//   RocmStorage::{allocate, from_host_f64,        theano::rocm::RocmStorage
//     to_host_f64} (storage.rs:31-99)
//   Tensor::to(&Device) / DType                   theano::DeviceTensor::from_host / to_host, to_dtype
//     (tensor.rs:277-299, dtype.rs:5-25)
//
// The reference's allocator and storage are mocks (no driver calls); these
// call hipMalloc / hipFree / hipMemcpyAsync and convert element types with
// libtq's tq_convert on the device.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <set>
#include <string>
#include <vector>

#include "theano_quantize.hpp"

namespace theano {

// DType (crates/theano-types/src/dtype.rs:5-25) without the complex and
// quantized variants; the values are tq.h's tq_dtype codes.
enum class DType : int { F16 = 0, BF16 = 1, F32 = 2, F64 = 3, U8 = 4, I8 = 5, I16 = 6, I32 = 7, I64 = 8, Bool = 9 };
size_t dtype_size(DType d);        // DType::size_in_bytes (dtype.rs:33-40)
const char* dtype_name(DType d);   // Display (dtype.rs:78-100)

namespace rocm {

// ------------------------------------------------------------ allocator

// allocator.rs:30-40: a range of device memory handed to a caller.
struct Block {
    void* ptr = nullptr;
    size_t size = 0;            // rounded size
    hipStream_t stream = nullptr;
};

// allocator.rs:42-59
struct AllocatorStats {
    size_t allocated_bytes = 0;
    size_t cached_bytes = 0;
    size_t peak_allocated_bytes = 0;
    size_t num_mallocs = 0;
    size_t num_frees = 0;
    size_t num_cache_hits = 0;
    size_t num_cache_misses = 0;
};

// Where segments come from: hipMalloc / hipFree on a device by default.
struct MemoryBackend {
    std::function<bool(void** ptr, size_t bytes)> malloc;  // false when out of memory
    std::function<void(void* ptr)> free;
    std::function<void()> synchronize;  // waits for work that may still use cached memory
};
MemoryBackend hip_backend(int device);

// Caching allocator (allocator.rs:61-305) with the reference's policy: small
// (<= 1 MB, rounded to 512 B) and large (rounded to 2 MB) pools, best-fit
// reuse, a cached block split when at least 512 B would remain, one driver
// allocation per miss, OOM recovery by releasing the cache and retrying once.
// On top of the reference: blocks are stream-ordered (a freed block is reused
// only by work on the stream it was allocated on, so no event is needed),
// adjacent free pieces of one driver segment merge back, and empty_cache()
// returns whole segments to the driver.
class CachingAllocator {
   public:
    static constexpr size_t kSmallPool = size_t(1) << 20;
    static constexpr size_t kMinBlock = 512;
    static constexpr size_t kSmallGranularity = 512;
    static constexpr size_t kLargeGranularity = size_t(2) << 20;

    explicit CachingAllocator(int device);
    CachingAllocator(int device, MemoryBackend backend);
    ~CachingAllocator();
    CachingAllocator(const CachingAllocator&) = delete;
    CachingAllocator& operator=(const CachingAllocator&) = delete;

    Result<Block> allocate(size_t size, hipStream_t stream = nullptr);
    void free(const Block& block);
    void empty_cache();
    AllocatorStats stats() const;
    int device() const { return device_; }
    static size_t round_size(size_t size);

   private:
    struct Piece;
    struct Segment;
    struct Key {
        hipStream_t stream;
        size_t size;
        uintptr_t ptr;
        bool operator<(const Key& o) const;
    };
    void insert_free(Piece* p);
    void erase_free(Piece* p);
    void release_segment(Segment* s);

    int device_;
    MemoryBackend backend_;
    mutable std::mutex mu_;
    std::set<Key> small_, large_;                  // free pieces, best fit per stream
    std::map<uintptr_t, Piece*> pieces_;           // every piece by address
    std::vector<std::unique_ptr<Segment>> segments_;
    AllocatorStats stats_;
};

// ------------------------------------------------------------ device

// device.rs:29-40, from hipGetDeviceProperties
struct DeviceProperties {
    std::string name;
    size_t total_memory = 0;
    uint32_t gcn_arch = 0;  // 950 for gfx950
    uint32_t multiprocessor_count = 0;
    uint32_t max_threads_per_block = 0;
    uint32_t max_threads_per_multiprocessor = 0;
    uint32_t warp_size = 0;
    size_t max_shared_memory_per_block = 0;
};

// device.rs:10-160: one GPU, its allocator and the pinned staging buffers of
// its host transfers.
class RocmDevice {
   public:
    static Result<std::shared_ptr<RocmDevice>> create(int ordinal);
    ~RocmDevice();
    int ordinal() const { return ordinal_; }
    const DeviceProperties& properties() const { return props_; }
    const std::string& name() const { return props_.name; }
    size_t total_memory() const { return props_.total_memory; }
    uint32_t gcn_arch() const { return props_.gcn_arch; }
    CachingAllocator& allocator() { return *alloc_; }
    Result<void> synchronize() const;
    // (free, total) device memory as the driver reports it
    Result<std::pair<size_t, size_t>> memory_info() const;
    void empty_cache() { alloc_->empty_cache(); }

    // host <-> device copies through two pinned staging buffers (chunks overlap
    // the host memcpy with the DMA); synchronous with respect to the host
    Result<void> copy_to_device(void* dst, const void* src, size_t bytes, hipStream_t stream);
    Result<void> copy_to_host(void* dst, const void* src, size_t bytes, hipStream_t stream);
    // D2H in staging-buffer chunks handed to `consume(chunk, offset, bytes)` on
    // the host while the next chunk's DMA runs (chunks are multiples of 8 bytes)
    Result<void> copy_to_host_chunks(const void* src, size_t bytes, hipStream_t stream,
                                     const std::function<void(const uint8_t*, size_t, size_t)>& consume);

   private:
    RocmDevice() = default;
    int ordinal_ = 0;
    DeviceProperties props_;
    std::unique_ptr<CachingAllocator> alloc_;
    std::mutex staging_mu_;
    void* staging_[2] = {nullptr, nullptr};
    hipEvent_t staged_[2] = {nullptr, nullptr};
};

// device.rs:162-213
class DeviceManager {
   public:
    static DeviceManager& global();
    Result<std::shared_ptr<RocmDevice>> get_device(int ordinal);
    int device_count() const;

   private:
    std::mutex mu_;
    std::vector<std::shared_ptr<RocmDevice>> devices_;
};

// ------------------------------------------------------------ storage

// storage.rs:11-99: `len` elements of `dtype` in a block of the device's
// caching allocator; the block goes back to the pool when the last copy of the
// storage is dropped.
class RocmStorage {
   public:
    static Result<RocmStorage> allocate(std::shared_ptr<RocmDevice> device, size_t len, DType dtype,
                                        hipStream_t stream = nullptr);
    // H2D of the f64 values, converted to `dtype` on the device (tq_convert)
    static Result<RocmStorage> from_host_f64(std::shared_ptr<RocmDevice> device, const double* data, size_t len,
                                             DType dtype, hipStream_t stream = nullptr);
    // D2H in the storage's own element type, widened to f64 on the host
    Result<std::vector<double>> to_host_f64() const;
    // a new storage holding the same values in `dtype` (tq_convert)
    Result<RocmStorage> to_dtype(DType dtype) const;

    RocmDevice& rocm_device() const { return *device_; }
    const std::shared_ptr<RocmDevice>& device_handle() const { return device_; }
    void* device_ptr() const { return block_ ? block_->ptr : nullptr; }
    size_t byte_size() const { return len_ * dtype_size(dtype_); }
    size_t len() const { return len_; }
    DType dtype() const { return dtype_; }
    hipStream_t stream() const { return stream_; }

   private:
    std::shared_ptr<RocmDevice> device_;
    std::shared_ptr<Block> block_;  // deleter returns the block to the allocator
    DType dtype_ = DType::F32;
    size_t len_ = 0;
    hipStream_t stream_ = nullptr;
};

}  // namespace rocm

// A tensor whose values stay in HBM between calls: Tensor::to(&Device::Rocm)
// (tensor.rs:277-299) without the per-call upload and download of the host
// Tensor API.  Dense, row-major.
class DeviceTensor {
   public:
    DeviceTensor() = default;
    DeviceTensor(rocm::RocmStorage storage, std::vector<size_t> shape);
    static Result<DeviceTensor> from_host(const Tensor& t, std::shared_ptr<rocm::RocmDevice> device, DType dtype,
                                          hipStream_t stream = nullptr);
    static Result<DeviceTensor> empty(std::shared_ptr<rocm::RocmDevice> device, std::vector<size_t> shape,
                                      DType dtype, hipStream_t stream = nullptr);
    Result<Tensor> to_host() const;
    Result<DeviceTensor> to_dtype(DType dtype) const;

    const std::vector<size_t>& shape() const { return shape_; }
    size_t numel() const;
    DType dtype() const { return storage_.dtype(); }
    void* data() const { return storage_.device_ptr(); }
    const rocm::RocmStorage& storage() const { return storage_; }
    hipStream_t stream() const { return storage_.stream(); }

   private:
    rocm::RocmStorage storage_;
    std::vector<size_t> shape_;
};

namespace nn {

// Device-resident forward of the quantized modules: x [M, in] (any float
// DType; converted on the device to the mode's activation type), y [M, out]
// F32, scratch from the device's caching allocator, everything on x's stream.
Result<DeviceTensor> forward(const QuantizedLinear& layer, const DeviceTensor& x);
Result<DeviceTensor> forward(const QuantizedMLP& mlp, const DeviceTensor& x);
// MultiheadAttention::forward_with_mask (transformer.rs:95-142): query, key,
// value [B, S, E] (one projection pass when the three share storage), mask
// [B or 1, (1,) S, S] additive; y [B, S, E] F32.
Result<DeviceTensor> forward_with_mask(const QuantizedMultiheadAttention& mha, const DeviceTensor& query,
                                       const DeviceTensor& key, const DeviceTensor& value,
                                       const std::optional<DeviceTensor>& mask);
Result<DeviceTensor> forward(const QuantizedMultiheadAttention& mha, const DeviceTensor& x);

}  // namespace nn
}  // namespace theano
