// Status text, per-stream workspaces and counters, and small host helpers of
// libanelm.
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
    d->num_cus = cus;
    d->id = id;
    return d;
}

__global__ void zero_u32_kernel(uint32_t* p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

// The state of (current device, stream), created on first use.  Its
// counters are zeroed by a fill kernel on the stream itself (ordered before
// every later launch there, and legal under stream capture).
StreamState* stream_state(hipStream_t stream) {
    Device* d = device();
    if (!d) return nullptr;
    std::lock_guard<std::mutex> lk(d->mu);
    for (StreamState* s : d->streams)
        if (s->stream == stream) return s;
    uint32_t* c = nullptr;
    hipError_t e = hipMalloc(&c, kCounterPool * sizeof(uint32_t));
    if (e != hipSuccess) { hip_fail(e, "hipMalloc(counters)"); return nullptr; }
    hipLaunchKernelGGL(zero_u32_kernel, dim3(64), dim3(256), 0, stream, c, kCounterPool);
    e = hipGetLastError();
    if (e != hipSuccess) {
        (void)hipFree(c);
        hip_fail(e, "zero_u32_kernel");
        return nullptr;
    }
    StreamState* s = new StreamState();
    s->stream = stream;
    s->counters = c;
    d->streams.push_back(s);
    return s;
}

// Grows one buffer of a stream's state.  Only work queued on that stream can
// still use the old buffer, so syncing that stream before the free suffices.
static void* grow(StreamState* s, void*& buf, size_t& have, size_t bytes) {
    std::lock_guard<std::mutex> lk(s->mu);
    if (bytes <= have) return buf;
    size_t want = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    want = (want + 0xffff) & ~size_t(0xffff);
    if (buf) {
        hipError_t e = hipStreamSynchronize(s->stream);
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
    StreamState* s = stream_state(stream);
    if (!s) return nullptr;
    return grow(s, s->ws, s->ws_bytes, bytes);
}

void* workspace2(size_t bytes, hipStream_t stream) {
    StreamState* s = stream_state(stream);
    if (!s) return nullptr;
    return grow(s, s->ws2, s->ws2_bytes, bytes);
}

uint32_t* counters(size_t n, CounterUser user, hipStream_t stream) {
    static_assert((size_t)kCtrUsers * kCounterRange <= kCounterPool, "counter ranges exceed the pool");
    if (n > kCounterRange) {
        set_error(ANELM_ERANGE, "%zu counters requested, a range holds %zu", n, kCounterRange);
        return nullptr;
    }
    StreamState* s = stream_state(stream);
    if (!s) return nullptr;
    return s->counters + (size_t)user * kCounterRange;
}

int stream_release(hipStream_t stream) {
    Device* d = device();
    if (!d) return ANELM_EHIP;
    StreamState* s = nullptr;
    {
        std::lock_guard<std::mutex> lk(d->mu);
        for (size_t i = 0; i < d->streams.size(); i++)
            if (d->streams[i]->stream == stream) {
                s = d->streams[i];
                d->streams.erase(d->streams.begin() + (long)i);
                break;
            }
    }
    if (!s) return ANELM_OK;
    hipError_t e = hipStreamSynchronize(stream);
    if (s->ws) (void)hipFree(s->ws);
    if (s->ws2) (void)hipFree(s->ws2);
    (void)hipFree(s->counters);
    delete s;
    if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
    return ANELM_OK;
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

int anelm_stream_release(void* stream) { return anelm::stream_release(anelm::as_stream(stream)); }

}  // extern "C"
