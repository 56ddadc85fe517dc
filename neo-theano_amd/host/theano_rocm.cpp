// theano_rocm.cpp -- caching allocator, device handle, storage and
// device-resident tensors (see theano_rocm.hpp).
#include "theano_rocm.hpp"

#include <algorithm>
#include <cctype>
#include <cmath>
#include <cstring>
#include <numeric>

namespace theano {

namespace {

template <class T, class F>
Result<T> capture(F&& f) {
    try {
        return f();
    } catch (const TheanoError& e) {
        return e;
    }
}

void check_hip(hipError_t e, const char* what) {
    if (e == hipErrorOutOfMemory) throw TheanoError::out_of_memory(std::string(what) + ": out of device memory");
    if (e != hipSuccess) throw TheanoError::runtime(std::string(what) + ": " + hipGetErrorString(e));
}

size_t numel_of(const std::vector<size_t>& shape) {
    return std::accumulate(shape.begin(), shape.end(), size_t{1}, [](size_t a, size_t b) { return a * b; });
}

// f16 / bf16 bit patterns -> f64 (exact)
double f16_to_f64(uint16_t h) {
    const double sign = (h & 0x8000) ? -1.0 : 1.0;
    const int e = (h >> 10) & 0x1F, f = h & 0x3FF;
    if (e == 0x1F) return f ? std::nan("") : sign * INFINITY;
    return e == 0 ? sign * std::ldexp(f, -24) : sign * std::ldexp(f | 0x400, e - 25);
}

double bf16_to_f64(uint16_t h) {
    const uint32_t u = static_cast<uint32_t>(h) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}

// n elements of a host buffer of `dtype` -> f64 (one tight loop per type)
template <class T, class F>
void widen_as(const uint8_t* p, size_t n, double* out, F f) {
    const T* v = reinterpret_cast<const T*>(p);  // staging chunks are page aligned
    for (size_t i = 0; i < n; ++i) out[i] = f(v[i]);
}

void widen(const uint8_t* p, DType d, size_t n, double* out) {
    switch (d) {
        case DType::F16: widen_as<uint16_t>(p, n, out, f16_to_f64); break;
        case DType::BF16: widen_as<uint16_t>(p, n, out, bf16_to_f64); break;
        case DType::F32: widen_as<float>(p, n, out, [](float v) { return static_cast<double>(v); }); break;
        case DType::F64: std::memcpy(out, p, n * 8); break;
        case DType::U8: widen_as<uint8_t>(p, n, out, [](uint8_t v) { return static_cast<double>(v); }); break;
        case DType::I8: widen_as<int8_t>(p, n, out, [](int8_t v) { return static_cast<double>(v); }); break;
        case DType::I16: widen_as<int16_t>(p, n, out, [](int16_t v) { return static_cast<double>(v); }); break;
        case DType::I32: widen_as<int32_t>(p, n, out, [](int32_t v) { return static_cast<double>(v); }); break;
        case DType::I64: widen_as<int64_t>(p, n, out, [](int64_t v) { return static_cast<double>(v); }); break;
        case DType::Bool: widen_as<uint8_t>(p, n, out, [](uint8_t v) { return v ? 1.0 : 0.0; }); break;
    }
}

constexpr size_t kStagingBytes = size_t(32) << 20;  // per pinned staging buffer

}  // namespace

size_t dtype_size(DType d) { return static_cast<size_t>(tq_dtype_size(static_cast<int>(d))); }

const char* dtype_name(DType d) {
    static const char* names[] = {"float16", "bfloat16", "float32", "float64", "uint8",
                                  "int8",    "int16",    "int32",   "int64",   "bool"};
    const int i = static_cast<int>(d);
    return (i >= 0 && i < 10) ? names[i] : "unknown";
}

namespace rocm {

// ------------------------------------------------------------ allocator

// A piece of a driver segment: allocated or free; neighbours by address.
struct CachingAllocator::Piece {
    uintptr_t ptr;
    size_t size;
    hipStream_t stream;
    bool allocated;
    Segment* segment;
    Piece* prev;
    Piece* next;
};

struct CachingAllocator::Segment {
    uintptr_t base;
    size_t size;
    bool small;  // pool of the request that created it
};

bool CachingAllocator::Key::operator<(const Key& o) const {
    if (stream != o.stream) return reinterpret_cast<uintptr_t>(stream) < reinterpret_cast<uintptr_t>(o.stream);
    if (size != o.size) return size < o.size;
    return ptr < o.ptr;
}

MemoryBackend hip_backend(int device) {
    MemoryBackend b;
    b.malloc = [device](void** p, size_t bytes) {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != device) (void)hipSetDevice(device);
        const hipError_t e = hipMalloc(p, bytes);
        if (cur != device) (void)hipSetDevice(cur);
        if (e != hipSuccess) {
            (void)hipGetLastError();  // clear the sticky error of a failed allocation
            return false;
        }
        return true;
    };
    b.free = [](void* p) { (void)hipFree(p); };
    b.synchronize = [device]() {
        int cur = 0;
        (void)hipGetDevice(&cur);
        if (cur != device) (void)hipSetDevice(device);
        (void)hipDeviceSynchronize();
        if (cur != device) (void)hipSetDevice(cur);
    };
    return b;
}

CachingAllocator::CachingAllocator(int device) : CachingAllocator(device, hip_backend(device)) {}

CachingAllocator::CachingAllocator(int device, MemoryBackend backend) : device_(device), backend_(std::move(backend)) {}

CachingAllocator::~CachingAllocator() {
    std::lock_guard<std::mutex> lk(mu_);
    if (!segments_.empty() && backend_.synchronize) backend_.synchronize();
    for (auto& s : segments_) backend_.free(reinterpret_cast<void*>(s->base));
    for (auto& kv : pieces_) delete kv.second;
}

size_t CachingAllocator::round_size(size_t size) {
    if (size <= kSmallPool) return (size + kSmallGranularity - 1) / kSmallGranularity * kSmallGranularity;
    return (size + kLargeGranularity - 1) / kLargeGranularity * kLargeGranularity;
}

void CachingAllocator::insert_free(Piece* p) {
    (p->size <= kSmallPool ? small_ : large_).insert(Key{p->stream, p->size, p->ptr});
}

void CachingAllocator::erase_free(Piece* p) {
    (p->size <= kSmallPool ? small_ : large_).erase(Key{p->stream, p->size, p->ptr});
}

Result<Block> CachingAllocator::allocate(size_t size, hipStream_t stream) {
    if (size == 0) return Block{nullptr, 0, stream};  // allocator.rs:89-96
    std::lock_guard<std::mutex> lk(mu_);
    const size_t rounded = round_size(size);
    const bool small = rounded <= kSmallPool;
    std::set<Key>& pool = small ? small_ : large_;
    auto it = pool.lower_bound(Key{stream, rounded, 0});
    if (it != pool.end() && it->stream == stream) {
        Piece* p = pieces_.at(it->ptr);
        pool.erase(it);
        if (p->size >= rounded + kMinBlock) {  // split: the remainder stays cached
            Piece* rest = new Piece{p->ptr + rounded, p->size - rounded, stream, false, p->segment, p, p->next};
            if (p->next) p->next->prev = rest;
            p->next = rest;
            p->size = rounded;
            pieces_[rest->ptr] = rest;
            insert_free(rest);
        }
        p->allocated = true;
        stats_.cached_bytes -= p->size;
        stats_.allocated_bytes += p->size;
        stats_.peak_allocated_bytes = std::max(stats_.peak_allocated_bytes, stats_.allocated_bytes);
        ++stats_.num_cache_hits;
        return Block{reinterpret_cast<void*>(p->ptr), p->size, stream};
    }
    // miss: one driver allocation of the rounded size; on failure release the
    // cache and retry once
    void* ptr = nullptr;
    if (!backend_.malloc(&ptr, rounded)) {
        if (backend_.synchronize) backend_.synchronize();
        for (size_t i = segments_.size(); i-- > 0;) {
            Segment* s = segments_[i].get();
            Piece* p = pieces_.at(s->base);
            if (!p->allocated && p->size == s->size) release_segment(s);
        }
        if (!backend_.malloc(&ptr, rounded))
            return TheanoError::out_of_memory("CachingAllocator::allocate: " + std::to_string(size) +
                                              " bytes on device " + std::to_string(device_));
    }
    ++stats_.num_mallocs;
    ++stats_.num_cache_misses;
    auto seg = std::make_unique<Segment>(Segment{reinterpret_cast<uintptr_t>(ptr), rounded, small});
    Piece* p = new Piece{seg->base, rounded, stream, true, seg.get(), nullptr, nullptr};
    pieces_[p->ptr] = p;
    segments_.push_back(std::move(seg));
    stats_.allocated_bytes += rounded;
    stats_.peak_allocated_bytes = std::max(stats_.peak_allocated_bytes, stats_.allocated_bytes);
    return Block{ptr, rounded, stream};
}

void CachingAllocator::free(const Block& block) {
    if (block.size == 0 || !block.ptr) return;  // allocator.rs:183-186
    std::lock_guard<std::mutex> lk(mu_);
    auto it = pieces_.find(reinterpret_cast<uintptr_t>(block.ptr));
    if (it == pieces_.end() || !it->second->allocated) return;  // not ours / already free
    Piece* p = it->second;
    p->allocated = false;
    stats_.allocated_bytes -= p->size;
    stats_.cached_bytes += p->size;
    // merge with free neighbours of the same segment
    if (p->next && !p->next->allocated) {
        Piece* n = p->next;
        erase_free(n);
        p->size += n->size;
        p->next = n->next;
        if (n->next) n->next->prev = p;
        pieces_.erase(n->ptr);
        delete n;
    }
    if (p->prev && !p->prev->allocated) {
        Piece* q = p->prev;
        erase_free(q);
        q->size += p->size;
        q->next = p->next;
        if (p->next) p->next->prev = q;
        pieces_.erase(p->ptr);
        delete p;
        p = q;
    }
    insert_free(p);
}

// Frees a segment whose single piece is free (caller holds the lock).
void CachingAllocator::release_segment(Segment* s) {
    Piece* p = pieces_.at(s->base);
    erase_free(p);
    pieces_.erase(p->ptr);
    delete p;
    stats_.cached_bytes -= s->size;
    ++stats_.num_frees;
    backend_.free(reinterpret_cast<void*>(s->base));
    segments_.erase(std::find_if(segments_.begin(), segments_.end(),
                                 [s](const std::unique_ptr<Segment>& u) { return u.get() == s; }));
}

void CachingAllocator::empty_cache() {
    std::lock_guard<std::mutex> lk(mu_);
    if (segments_.empty()) return;
    if (backend_.synchronize) backend_.synchronize();
    for (size_t i = segments_.size(); i-- > 0;) {
        Segment* s = segments_[i].get();
        Piece* p = pieces_.at(s->base);
        if (!p->allocated && p->size == s->size) release_segment(s);
    }
}

AllocatorStats CachingAllocator::stats() const {
    std::lock_guard<std::mutex> lk(mu_);
    return stats_;
}

// ------------------------------------------------------------ device

Result<std::shared_ptr<RocmDevice>> RocmDevice::create(int ordinal) {
    return capture<std::shared_ptr<RocmDevice>>([&]() -> Result<std::shared_ptr<RocmDevice>> {
        int count = 0;
        check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount");
        if (ordinal < 0 || ordinal >= count)
            return TheanoError::invalid_argument("RocmDevice: ordinal " + std::to_string(ordinal) + " of " +
                                                 std::to_string(count) + " devices");
        hipDeviceProp_t p;
        check_hip(hipGetDeviceProperties(&p, ordinal), "hipGetDeviceProperties");
        std::shared_ptr<RocmDevice> d(new RocmDevice());
        d->ordinal_ = ordinal;
        d->props_.name = p.name;
        d->props_.total_memory = p.totalGlobalMem;
        // "gfx950[:features]" -> 950; a name with a letter digit (gfx90a) reads as hexadecimal
        const std::string arch = std::string(p.gcnArchName).substr(0, std::string(p.gcnArchName).find(':'));
        const std::string num = arch.size() > 3 ? arch.substr(3) : std::string("0");
        const bool decimal = std::all_of(num.begin(), num.end(), [](char c) { return c >= '0' && c <= '9'; });
        const uint32_t g = static_cast<uint32_t>(std::stoul(num, nullptr, decimal ? 10 : 16));
        d->props_.gcn_arch = g;
        d->props_.multiprocessor_count = static_cast<uint32_t>(p.multiProcessorCount);
        d->props_.max_threads_per_block = static_cast<uint32_t>(p.maxThreadsPerBlock);
        d->props_.max_threads_per_multiprocessor = static_cast<uint32_t>(p.maxThreadsPerMultiProcessor);
        d->props_.warp_size = static_cast<uint32_t>(p.warpSize);
        d->props_.max_shared_memory_per_block = p.sharedMemPerBlock;
        d->alloc_ = std::make_unique<CachingAllocator>(ordinal);
        return d;
    });
}

RocmDevice::~RocmDevice() {
    for (int i = 0; i < 2; ++i) {
        if (staged_[i]) (void)hipEventDestroy(staged_[i]);
        if (staging_[i]) (void)hipHostFree(staging_[i]);
    }
}

Result<void> RocmDevice::synchronize() const {
    return capture<void>([&]() -> Result<void> {
        int cur = 0;
        check_hip(hipGetDevice(&cur), "hipGetDevice");
        check_hip(hipSetDevice(ordinal_), "hipSetDevice");
        const hipError_t e = hipDeviceSynchronize();
        (void)hipSetDevice(cur);
        check_hip(e, "hipDeviceSynchronize");
        return {};
    });
}

Result<std::pair<size_t, size_t>> RocmDevice::memory_info() const {
    return capture<std::pair<size_t, size_t>>([&]() -> Result<std::pair<size_t, size_t>> {
        int cur = 0;
        check_hip(hipGetDevice(&cur), "hipGetDevice");
        check_hip(hipSetDevice(ordinal_), "hipSetDevice");
        size_t free_b = 0, total = 0;
        const hipError_t e = hipMemGetInfo(&free_b, &total);
        (void)hipSetDevice(cur);
        check_hip(e, "hipMemGetInfo");
        return std::make_pair(free_b, total);
    });
}

// Chunks of up to kStagingBytes alternate between the two pinned buffers: the
// host memcpy into one overlaps the DMA out of the other; an event per buffer
// says when its previous DMA has finished.
Result<void> RocmDevice::copy_to_device(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    return capture<void>([&]() -> Result<void> {
        std::lock_guard<std::mutex> lk(staging_mu_);
        for (int i = 0; i < 2; ++i) {
            if (!staging_[i]) check_hip(hipHostMalloc(&staging_[i], kStagingBytes, hipHostMallocDefault), "hipHostMalloc");
            if (!staged_[i]) check_hip(hipEventCreateWithFlags(&staged_[i], hipEventDisableTiming), "hipEventCreate");
        }
        size_t off = 0;
        for (int b = 0; off < bytes; b ^= 1) {
            const size_t n = std::min(kStagingBytes, bytes - off);
            check_hip(hipEventSynchronize(staged_[b]), "staging wait");
            std::memcpy(staging_[b], static_cast<const uint8_t*>(src) + off, n);
            check_hip(hipMemcpyAsync(static_cast<uint8_t*>(dst) + off, staging_[b], n, hipMemcpyHostToDevice, stream),
                      "hipMemcpyAsync H2D");
            check_hip(hipEventRecord(staged_[b], stream), "hipEventRecord");
            off += n;
        }
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
        return {};
    });
}

Result<void> RocmDevice::copy_to_host(void* dst, const void* src, size_t bytes, hipStream_t stream) {
    return copy_to_host_chunks(src, bytes, stream, [dst](const uint8_t* chunk, size_t off, size_t n) {
        std::memcpy(static_cast<uint8_t*>(dst) + off, chunk, n);
    });
}

Result<void> RocmDevice::copy_to_host_chunks(const void* src, size_t bytes, hipStream_t stream,
                                             const std::function<void(const uint8_t*, size_t, size_t)>& consume) {
    return capture<void>([&]() -> Result<void> {
        std::lock_guard<std::mutex> lk(staging_mu_);
        for (int i = 0; i < 2; ++i) {
            if (!staging_[i]) check_hip(hipHostMalloc(&staging_[i], kStagingBytes, hipHostMallocDefault), "hipHostMalloc");
            if (!staged_[i]) check_hip(hipEventCreateWithFlags(&staged_[i], hipEventDisableTiming), "hipEventCreate");
        }
        // DMA chunk c into buffer c % 2 while the host consumes chunk c - 1
        const size_t chunks = (bytes + kStagingBytes - 1) / kStagingBytes;
        auto issue = [&](size_t c) {
            const size_t off = c * kStagingBytes, n = std::min(kStagingBytes, bytes - off);
            check_hip(hipMemcpyAsync(staging_[c & 1], static_cast<const uint8_t*>(src) + off, n,
                                     hipMemcpyDeviceToHost, stream),
                      "hipMemcpyAsync D2H");
            check_hip(hipEventRecord(staged_[c & 1], stream), "hipEventRecord");
        };
        if (chunks) issue(0);
        for (size_t c = 0; c < chunks; ++c) {
            if (c + 1 < chunks) issue(c + 1);
            check_hip(hipEventSynchronize(staged_[c & 1]), "staging wait");
            const size_t off = c * kStagingBytes, n = std::min(kStagingBytes, bytes - off);
            consume(static_cast<const uint8_t*>(staging_[c & 1]), off, n);
        }
        return {};
    });
}

DeviceManager& DeviceManager::global() {
    static DeviceManager m;
    return m;
}

Result<std::shared_ptr<RocmDevice>> DeviceManager::get_device(int ordinal) {
    std::lock_guard<std::mutex> lk(mu_);
    if (ordinal < 0) return TheanoError::invalid_argument("DeviceManager: negative ordinal");
    if (static_cast<size_t>(ordinal) < devices_.size() && devices_[ordinal]) return devices_[ordinal];
    auto d = RocmDevice::create(ordinal);
    if (d.is_err()) return d.unwrap_err();
    if (devices_.size() <= static_cast<size_t>(ordinal)) devices_.resize(ordinal + 1);
    devices_[ordinal] = d.unwrap();
    return devices_[ordinal];
}

int DeviceManager::device_count() const {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

// ------------------------------------------------------------ storage

Result<RocmStorage> RocmStorage::allocate(std::shared_ptr<RocmDevice> device, size_t len, DType dtype,
                                          hipStream_t stream) {
    if (!device) return TheanoError::invalid_argument("RocmStorage::allocate: no device");
    const size_t es = dtype_size(dtype);
    if (es == 0) return TheanoError::invalid_argument("RocmStorage::allocate: unsupported dtype");
    auto b = device->allocator().allocate(len * es, stream);
    if (b.is_err()) return b.unwrap_err();
    RocmStorage s;
    s.device_ = device;
    s.block_ = std::shared_ptr<Block>(new Block(b.unwrap()), [device](Block* blk) {
        device->allocator().free(*blk);
        delete blk;
    });
    s.dtype_ = dtype;
    s.len_ = len;
    s.stream_ = stream;
    return s;
}

Result<RocmStorage> RocmStorage::from_host_f64(std::shared_ptr<RocmDevice> device, const double* data, size_t len,
                                               DType dtype, hipStream_t stream) {
    auto r = allocate(device, len, dtype, stream);
    if (r.is_err() || len == 0) return r;
    RocmStorage s = std::move(r).unwrap();
    if (dtype == DType::F64) {
        auto c = device->copy_to_device(s.device_ptr(), data, len * 8, stream);
        if (c.is_err()) return c.unwrap_err();
        return s;
    }
    auto staging = allocate(device, len, DType::F64, stream);  // f64 values, converted on the device
    if (staging.is_err()) return staging.unwrap_err();
    RocmStorage st = std::move(staging).unwrap();
    auto c = device->copy_to_device(st.device_ptr(), data, len * 8, stream);
    if (c.is_err()) return c.unwrap_err();
    const int rc = tq_convert(st.device_ptr(), TQ_DT_F64, s.device_ptr(), static_cast<int>(dtype),
                              static_cast<int64_t>(len), reinterpret_cast<tq_stream_t>(stream));
    if (rc != TQ_OK) return TheanoError::from_status(rc, "RocmStorage::from_host_f64");
    return s;  // the staging block returns to the pool in stream order
}

Result<std::vector<double>> RocmStorage::to_host_f64() const {
    std::vector<double> out(len_);
    if (len_ == 0) return out;
    if (dtype_ == DType::F64) {  // straight into the result
        auto c = device_->copy_to_host(out.data(), device_ptr(), byte_size(), stream_);
        if (c.is_err()) return c.unwrap_err();
        return out;
    }
    const size_t es = dtype_size(dtype_);
    auto c = device_->copy_to_host_chunks(device_ptr(), byte_size(), stream_,
                                          [&](const uint8_t* chunk, size_t off, size_t n) {
                                              widen(chunk, dtype_, n / es, out.data() + off / es);
                                          });
    if (c.is_err()) return c.unwrap_err();
    return out;
}

Result<RocmStorage> RocmStorage::to_dtype(DType dtype) const {
    auto r = allocate(device_, len_, dtype, stream_);
    if (r.is_err() || len_ == 0) return r;
    RocmStorage s = std::move(r).unwrap();
    const int rc = tq_convert(device_ptr(), static_cast<int>(dtype_), s.device_ptr(), static_cast<int>(dtype),
                              static_cast<int64_t>(len_), reinterpret_cast<tq_stream_t>(stream_));
    if (rc != TQ_OK) return TheanoError::from_status(rc, "RocmStorage::to_dtype");
    return s;
}

}  // namespace rocm

// ------------------------------------------------------------ DeviceTensor

DeviceTensor::DeviceTensor(rocm::RocmStorage storage, std::vector<size_t> shape)
    : storage_(std::move(storage)), shape_(std::move(shape)) {}

size_t DeviceTensor::numel() const { return numel_of(shape_); }

Result<DeviceTensor> DeviceTensor::from_host(const Tensor& t, std::shared_ptr<rocm::RocmDevice> device, DType dtype,
                                             hipStream_t stream) {
    auto s = rocm::RocmStorage::from_host_f64(std::move(device), t.data(), t.numel(), dtype, stream);
    if (s.is_err()) return s.unwrap_err();
    return DeviceTensor(std::move(s).unwrap(), t.shape());
}

Result<DeviceTensor> DeviceTensor::empty(std::shared_ptr<rocm::RocmDevice> device, std::vector<size_t> shape,
                                         DType dtype, hipStream_t stream) {
    auto s = rocm::RocmStorage::allocate(std::move(device), numel_of(shape), dtype, stream);
    if (s.is_err()) return s.unwrap_err();
    return DeviceTensor(std::move(s).unwrap(), std::move(shape));
}

Result<Tensor> DeviceTensor::to_host() const {
    auto v = storage_.to_host_f64();
    if (v.is_err()) return v.unwrap_err();
    return Tensor::from_slice(std::move(v).unwrap(), shape_);
}

Result<DeviceTensor> DeviceTensor::to_dtype(DType dtype) const {
    if (dtype == this->dtype()) return *this;
    auto s = storage_.to_dtype(dtype);
    if (s.is_err()) return s.unwrap_err();
    return DeviceTensor(std::move(s).unwrap(), shape_);
}

namespace nn {

namespace {

Result<std::pair<size_t, size_t>> rows_of(const DeviceTensor& x, size_t in, const char* what) {
    const auto& sh = x.shape();
    if (sh.empty() || sh.size() > 2 || sh.back() != in)
        return TheanoError::shape_mismatch(std::string(what) + ": expected [*, " + std::to_string(in) + "] input");
    if (!x.storage().device_handle()) return TheanoError::invalid_argument(std::string(what) + ": empty tensor");
    return std::make_pair(sh.size() == 2 ? sh[0] : size_t{1}, in);
}

}  // namespace

Result<DeviceTensor> forward(const QuantizedLinear& layer, const DeviceTensor& x) {
    auto rk = rows_of(x, layer.in_features(), "QuantizedLinear::forward");
    if (rk.is_err()) return rk.unwrap_err();
    const size_t m = rk.unwrap().first, k = layer.in_features(), n = layer.out_features();
    const auto dev = x.storage().device_handle();
    const hipStream_t st = x.stream();
    const DType act = layer.mode() == QuantizedLinear::Mode::W4 ? DType::BF16 : DType::F32;
    auto xa = x.to_dtype(act);
    if (xa.is_err()) return xa.unwrap_err();
    std::vector<size_t> yshape = x.shape();
    yshape.back() = n;
    auto y = DeviceTensor::empty(dev, yshape, DType::F32, st);
    if (y.is_err()) return y.unwrap_err();
    std::optional<rocm::RocmStorage> codes, scales, ws;
    const bool quant_act = layer.mode() == QuantizedLinear::Mode::W8A8 || layer.mode() == QuantizedLinear::Mode::FP8;
    if (quant_act) {
        auto c = rocm::RocmStorage::allocate(dev, m * k, DType::I8, st);
        auto s = rocm::RocmStorage::allocate(dev, m, DType::F32, st);
        if (c.is_err()) return c.unwrap_err();
        if (s.is_err()) return s.unwrap_err();
        codes = std::move(c).unwrap();
        scales = std::move(s).unwrap();
    }
    const size_t wsb = layer.workspace_bytes(static_cast<int64_t>(m));
    if (wsb) {
        auto w = rocm::RocmStorage::allocate(dev, wsb, DType::U8, st);
        if (w.is_err()) return w.unwrap_err();
        ws = std::move(w).unwrap();
    }
    auto r = layer.forward_device(xa.unwrap().data(), static_cast<int64_t>(m), static_cast<float*>(y.unwrap().data()),
                                  st, codes ? static_cast<int8_t*>(codes->device_ptr()) : nullptr,
                                  scales ? static_cast<float*>(scales->device_ptr()) : nullptr,
                                  ws ? ws->device_ptr() : nullptr, wsb);
    if (r.is_err()) return r.unwrap_err();
    return y;  // scratch storages return to the pool in stream order
}

Result<DeviceTensor> forward(const QuantizedMLP& mlp, const DeviceTensor& x) {
    auto rk = rows_of(x, mlp.hidden(), "QuantizedMLP::forward");
    if (rk.is_err()) return rk.unwrap_err();
    const size_t m = rk.unwrap().first;
    const auto dev = x.storage().device_handle();
    const hipStream_t st = x.stream();
    auto xb = x.to_dtype(DType::BF16);
    if (xb.is_err()) return xb.unwrap_err();
    auto y = DeviceTensor::empty(dev, x.shape(), DType::F32, st);
    if (y.is_err()) return y.unwrap_err();
    const size_t wsb = mlp.workspace_bytes(static_cast<int64_t>(m));
    auto ws = rocm::RocmStorage::allocate(dev, std::max<size_t>(wsb, 1), DType::U8, st);
    if (ws.is_err()) return ws.unwrap_err();
    auto r = mlp.forward_device(static_cast<const uint16_t*>(xb.unwrap().data()), static_cast<int64_t>(m),
                                ws.unwrap().device_ptr(), wsb, static_cast<float*>(y.unwrap().data()), st);
    if (r.is_err()) return r.unwrap_err();
    return y;
}

Result<DeviceTensor> forward_with_mask(const QuantizedMultiheadAttention& mha, const DeviceTensor& query,
                                       const DeviceTensor& key, const DeviceTensor& value,
                                       const std::optional<DeviceTensor>& mask) {
    const size_t e = mha.embed_dim();
    const auto& sh = query.shape();
    if (sh.size() != 3 || sh[2] != e || key.shape() != sh || value.shape() != sh)
        return TheanoError::shape_mismatch("QuantizedMultiheadAttention::forward: query, key, value must be [batch, seq, " +
                                           std::to_string(e) + "]");
    if (!query.storage().device_handle() || !key.storage().device_handle() || !value.storage().device_handle())
        return TheanoError::invalid_argument("QuantizedMultiheadAttention::forward: empty tensor");
    const size_t b = sh[0], s = sh[1], m = b * s;
    int64_t mb = 0;
    std::optional<DeviceTensor> mf;
    if (mask) {
        const auto& ms = mask->shape();
        const bool ok3 = ms.size() == 3 && ms[1] == s && ms[2] == s;
        const bool ok4 = ms.size() == 4 && ms[1] == 1 && ms[2] == s && ms[3] == s;
        if (!(ok3 || ok4) || (ms[0] != 1 && ms[0] != b))
            return TheanoError::shape_mismatch("QuantizedMultiheadAttention::forward: mask must be [batch or 1, (1,) seq, seq]");
        auto c = mask->to_dtype(DType::F32);
        if (c.is_err()) return c.unwrap_err();
        mf = std::move(c).unwrap();
        mb = static_cast<int64_t>(ms[0]);
    }
    const auto dev = query.storage().device_handle();
    const hipStream_t st = query.stream();
    // the fused projection once for self-attention, per input otherwise; each [m, 3E]
    const bool self = query.data() == key.data() && key.data() == value.data() && query.dtype() == key.dtype() &&
                      key.dtype() == value.dtype();
    std::vector<DeviceTensor> proj;
    for (const DeviceTensor* in : self ? std::vector<const DeviceTensor*>{&query}
                                       : std::vector<const DeviceTensor*>{&query, &key, &value}) {
        auto y = forward(mha.qkv(), DeviceTensor(in->storage(), {m, e}));
        if (y.is_err()) return y.unwrap_err();
        proj.push_back(std::move(y).unwrap());
    }
    const float* qp = static_cast<const float*>(proj[0].data());
    const float* kp = static_cast<const float*>(proj[self ? 0 : 1].data()) + e;
    const float* vp = static_cast<const float*>(proj[self ? 0 : 2].data()) + 2 * e;
    auto att = DeviceTensor::empty(dev, {m, e}, DType::F32, st);
    if (att.is_err()) return att.unwrap_err();
    const int64_t ld = static_cast<int64_t>(3 * e);
    const int rc = tq_attention_f32(qp, ld, kp, ld, vp, ld, mf ? static_cast<const float*>(mf->data()) : nullptr, mb,
                                    static_cast<int64_t>(b), static_cast<int64_t>(s),
                                    static_cast<int64_t>(mha.num_heads()), static_cast<int64_t>(mha.head_dim()),
                                    static_cast<float*>(att.unwrap().data()), static_cast<int64_t>(e),
                                    reinterpret_cast<tq_stream_t>(st));
    if (rc != TQ_OK) return TheanoError::from_status(rc, "QuantizedMultiheadAttention attention");
    auto y = forward(mha.out_proj(), att.unwrap());
    if (y.is_err()) return y.unwrap_err();
    return DeviceTensor(y.unwrap().storage(), sh);
}

Result<DeviceTensor> forward(const QuantizedMultiheadAttention& mha, const DeviceTensor& x) {
    return forward_with_mask(mha, x, x, x, std::nullopt);
}

}  // namespace nn
}  // namespace theano
