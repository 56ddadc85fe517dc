// tq_api.hip -- host-only parts of the C ABI: status strings, thread-local
// error messages, QuantDType ranges and the observers' scalar scale math.
#include <cmath>
#include <cstring>

#include "tq_internal.h"

namespace tq {

namespace {
thread_local char g_last_error[512] = "";
}

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
    va_end(ap);
    return status;
}

void clear_error() { g_last_error[0] = '\0'; }

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(TQ_EHIP, "%s: %s", what, hipGetErrorString(e));
    return TQ_OK;
}

int device_cu_count() {
    // one slot per device; concurrent first calls store the same value
    static std::atomic<int> cached[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int cus = cached[dev].load(std::memory_order_relaxed);
    if (cus == 0) {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            cus <= 0)
            cus = 256;
        cached[dev].store(cus, std::memory_order_relaxed);
    }
    return cus;
}

int allow_dynamic_lds(const void* kernel, int bytes, std::atomic<uint64_t>& done_devices) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return fail(TQ_EHIP, "hipGetDevice failed");
    const uint64_t bit = uint64_t{1} << dev;
    if (done_devices.load(std::memory_order_acquire) & bit) return TQ_OK;
    // idempotent: threads racing here all set the same attribute
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes) != hipSuccess)
        return fail(TQ_EHIP, "hipFuncSetAttribute(MaxDynamicSharedMemorySize, %d) failed", bytes);
    done_devices.fetch_or(bit, std::memory_order_acq_rel);
    return TQ_OK;
}

}  // namespace tq

extern "C" {

int tq_version(void) { return 100; }

const char* tq_status_string(int status) {
    switch (status) {
    case TQ_OK: return "TQ_OK";
    case TQ_EINVAL: return "TQ_EINVAL";
    case TQ_EHIP: return "TQ_EHIP";
    case TQ_ENOMEM: return "TQ_ENOMEM";
    default: return "TQ_UNKNOWN";
    }
}

const char* tq_last_error(void) { return tq::g_last_error; }

// QuantDType::{bits, is_signed, qmin, qmax}: crates/theano-quantize/src/qconfig.rs:12-41
int tq_qdtype_info(int qdtype, int* bits, int* is_signed, double* qmin, double* qmax) {
    static const int kBits[4] = {8, 8, 4, 8};
    static const int kSigned[4] = {1, 0, 1, 0};
    static const double kMin[4] = {-128.0, 0.0, -8.0, -448.0};
    static const double kMax[4] = {127.0, 255.0, 7.0, 448.0};
    if (qdtype < 0 || qdtype > 3) return tq::fail(TQ_EINVAL, "unknown QuantDType %d", qdtype);
    if (bits) *bits = kBits[qdtype];
    if (is_signed) *is_signed = kSigned[qdtype];
    if (qmin) *qmin = kMin[qdtype];
    if (qmax) *qmax = kMax[qdtype];
    return TQ_OK;
}

// Observer::compute_scale_zero_point for one {min, max} pair:
// crates/theano-quantize/src/observer.rs:51-66 (and :93-106 per channel).
int tq_observer_scale_zp(double min_val, double max_val, int initialized, int qdtype,
                         double* scale, double* zero_point) {
    double qmin = 0, qmax = 0;
    const int st = tq_qdtype_info(qdtype, nullptr, nullptr, &qmin, &qmax);
    if (st != TQ_OK) return st;
    if (!scale || !zero_point) return tq::fail(TQ_EINVAL, "null output pointer");
    if (!initialized) {
        *scale = 1.0;
        *zero_point = 0.0;
        return TQ_OK;
    }
    volatile double s = (max_val - min_val) / (qmax - qmin);  // no contraction
    double sc = std::fmax(s, 1e-10);
    volatile double z = qmin - min_val / sc;
    double zr = std::round(z);
    if (zr < qmin) zr = qmin;  // Rust f64::clamp keeps NaN
    if (zr > qmax) zr = qmax;
    *scale = sc;
    *zero_point = zr;
    return TQ_OK;
}

}  // extern "C"
