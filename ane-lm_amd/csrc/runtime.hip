// Status text, per-device workspace and small host helpers of libanelm.
#include "anelm_internal.hpp"

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <mutex>

namespace anelm {

static thread_local char g_err[512] = "";

int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what) {
    return set_error(ANELM_EHIP, "%s failed: %s", what, hipGetErrorString(e));
}

static constexpr int kMaxDevices = 64;
static Device g_dev[kMaxDevices];
static std::mutex g_mu;

Device* device() {
    int id = 0;
    hipError_t e = hipGetDevice(&id);
    if (e != hipSuccess) { hip_fail(e, "hipGetDevice"); return nullptr; }
    if (id < 0 || id >= kMaxDevices) { set_error(ANELM_ERANGE, "device %d out of range", id); return nullptr; }
    Device* d = &g_dev[id];
    if (d->id == id) return d;
    std::lock_guard<std::mutex> lk(g_mu);
    if (d->id == id) return d;
    int cus = 0;
    e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, id);
    if (e != hipSuccess) { hip_fail(e, "hipDeviceGetAttribute"); return nullptr; }
    uint32_t* c = nullptr;
    e = hipMalloc(&c, kCounterPool * sizeof(uint32_t));
    if (e != hipSuccess) { hip_fail(e, "hipMalloc(counters)"); return nullptr; }
    e = hipMemset(c, 0, kCounterPool * sizeof(uint32_t));
    if (e != hipSuccess) { hip_fail(e, "hipMemset(counters)"); return nullptr; }
    e = hipDeviceSynchronize();
    if (e != hipSuccess) { hip_fail(e, "hipDeviceSynchronize"); return nullptr; }
    d->num_cus = cus;
    d->counters = c;
    d->n_counters = kCounterPool;
    d->id = id;
    return d;
}

static void* grow(void*& buf, size_t& have, size_t bytes, hipStream_t stream) {
    if (bytes <= have) return buf;
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    want = (want + 0xffff) & ~size_t(0xffff);
    if (buf) {
        hipError_t e = hipStreamSynchronize(stream);
        if (e != hipSuccess) { hip_fail(e, "hipStreamSynchronize"); return nullptr; }
        e = hipFree(buf);
        if (e != hipSuccess) { hip_fail(e, "hipFree(workspace)"); return nullptr; }
        buf = nullptr;
        have = 0;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, want);
    if (e != hipSuccess) {
        set_error(ANELM_ENOMEM, "workspace of %zu bytes: %s", want, hipGetErrorString(e));
        return nullptr;
    }
    buf = p;
    have = want;
    return p;
}

void* workspace(size_t bytes, hipStream_t stream) {
    Device* d = device();
    if (!d) return nullptr;
    return grow(d->ws, d->ws_bytes, bytes, stream);
}

void* workspace2(size_t bytes, hipStream_t stream) {
    Device* d = device();
    if (!d) return nullptr;
    return grow(d->ws2, d->ws2_bytes, bytes, stream);
}

uint32_t* counters(size_t n, CounterUser user) {
    static_assert((size_t)kCtrUsers * kCounterRange <= kCounterPool, "counter ranges exceed the pool");
    Device* d = device();
    if (!d) return nullptr;
    if (n > kCounterRange) {
        set_error(ANELM_ERANGE, "%zu counters requested, a range holds %zu", n, kCounterRange);
        return nullptr;
    }
    return d->counters + (size_t)user * kCounterRange;
}

void rope_row(float* cos_out, float* sin_out, int rot_dim, int pos, float theta) {
    for (int i = 0, j = 0; i < rot_dim; i += 2, j++) {
        float freq = 1.0f / powf(theta, (float)i / (float)rot_dim);
        float angle = (float)pos * freq;
        cos_out[j] = cosf(angle);
        sin_out[j] = sinf(angle);
    }
}

}  // namespace anelm

extern "C" {

const char* anelm_last_error(void) { return anelm::g_err; }

int anelm_version(void) { return 1; }

int anelm_device_cus(void) {
    anelm::Device* d = anelm::device();
    return d ? d->num_cus : 0;
}

}  // extern "C"
