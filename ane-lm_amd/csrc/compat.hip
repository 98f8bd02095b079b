// Host-pointer, synchronous forms of the core/cpu_ops.h functions
// (declared in include/anelm_cpu_ops.h).  Each call stages its operands into
// per-device staging buffers, runs the native kernel on the null stream, and
// copies results back, so the semantics match the reference's in-place host
// functions (core/cpu_ops.cpp:6-204).
#include "anelm_internal.hpp"
#include "../../include/anelm_cpu_ops.h"

#include <mutex>

namespace anelm {
namespace {

constexpr int kSlots = 8;

struct Staging {
    int dev = -1;
    void* p[kSlots] = {};
    size_t n[kSlots] = {};
};

std::mutex g_stage_mu;
Staging g_stage[64];

// Device buffer `slot` of at least `bytes` on the current device.
void* slot_ptr(int slot, size_t bytes) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
        set_error(ANELM_EHIP, "no current HIP device");
        return nullptr;
    }
    Staging& s = g_stage[dev];
    if (bytes == 0) bytes = 4;
    if (s.n[slot] >= bytes) return s.p[slot];
    if (s.p[slot]) (void)hipFree(s.p[slot]);
    s.p[slot] = nullptr;
    s.n[slot] = 0;
    const size_t want = (bytes + 4095) & ~size_t(4095);
    hipError_t e = hipMalloc(&s.p[slot], want);
    if (e != hipSuccess) {
        set_error(ANELM_ENOMEM, "staging %zu bytes: %s", want, hipGetErrorString(e));
        s.p[slot] = nullptr;
        return nullptr;
    }
    s.n[slot] = want;
    return s.p[slot];
}

struct Stage {
    std::lock_guard<std::mutex> lk{g_stage_mu};
    int rc = ANELM_OK;
    template <typename T>
    T* in(int slot, const T* host, size_t count) {
        if (rc) return nullptr;
        T* d = static_cast<T*>(slot_ptr(slot, count * sizeof(T)));
        if (!d) { rc = ANELM_ENOMEM; return nullptr; }
        if (host && count) {
            hipError_t e = hipMemcpy(d, host, count * sizeof(T), hipMemcpyHostToDevice);
            if (e != hipSuccess) { rc = hip_fail(e, "hipMemcpy H2D"); return nullptr; }
        }
        return d;
    }
    template <typename T>
    int out(T* host, const T* dev, size_t count) {
        if (rc) return rc;
        hipError_t e = hipMemcpy(host, dev, count * sizeof(T), hipMemcpyDeviceToHost);
        if (e != hipSuccess) rc = hip_fail(e, "hipMemcpy D2H");
        return rc;
    }
    int run(int code) {
        if (rc) return rc;
        if (code) { rc = code; return rc; }
        hipError_t e = hipDeviceSynchronize();
        if (e != hipSuccess) rc = hip_fail(e, "hipDeviceSynchronize");
        return rc;
    }
};

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" {

int anelm_cpu_silu_vec_inplace(float* x, int n, float* tmp) {
    (void)tmp;
    ANELM_NONNULL(x);
    ANELM_REQUIRE(n >= 0, "silu_vec_inplace: n %d", n);
    Stage s;
    float* dx = s.in(0, x, (size_t)n);
    if (s.run(dx ? anelm_silu_inplace(dx, n, nullptr) : s.rc)) return s.rc;
    return s.out(x, dx, (size_t)n);
}

int anelm_cpu_mul_sigmoid_inplace(float* y, const float* z, int n, float* tmp) {
    (void)tmp;
    ANELM_NONNULL(y);
    ANELM_NONNULL(z);
    ANELM_REQUIRE(n >= 0, "mul_sigmoid_inplace: n %d", n);
    Stage s;
    float* dy = s.in(0, y, (size_t)n);
    float* dz = s.in(1, z, (size_t)n);
    if (s.run(dz ? anelm_mul_sigmoid_inplace(dy, dz, n, nullptr) : s.rc)) return s.rc;
    return s.out(y, dy, (size_t)n);
}

int anelm_cpu_rmsnorm(float* out, const float* x, const float* weight, int dim, float eps) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(x);
    ANELM_NONNULL(weight);
    ANELM_REQUIRE(dim > 0, "rmsnorm: dim %d", dim);
    Stage s;
    float* dx = s.in(0, x, (size_t)dim);
    float* dw = s.in(1, weight, (size_t)dim);
    if (s.run(dw ? anelm_rmsnorm(dx, dx, dw, dim, 1, dim, dim, eps, nullptr) : s.rc)) return s.rc;
    return s.out(out, dx, (size_t)dim);
}

int anelm_cpu_rmsnorm_gated(float* out, const float* x, const float* z, const float* weight, int dim) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(x);
    ANELM_NONNULL(z);
    ANELM_NONNULL(weight);
    ANELM_REQUIRE(dim > 0, "rmsnorm_gated: dim %d", dim);
    Stage s;
    float* dx = s.in(0, x, (size_t)dim);
    float* dz = s.in(1, z, (size_t)dim);
    float* dw = s.in(2, weight, (size_t)dim);
    float* dout = s.in<float>(3, nullptr, (size_t)dim);
    if (s.run(dout ? anelm_rmsnorm_gated(dout, dx, dz, dw, dim, 1, nullptr) : s.rc)) return s.rc;
    return s.out(out, dout, (size_t)dim);
}

int anelm_cpu_apply_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                                int q_head_stride, int k_head_stride, int rot_dim, int pos,
                                float theta, const float* cos_row, const float* sin_row) {
    ANELM_REQUIRE(n_q_heads >= 0 && n_kv_heads >= 0 && head_dim > 0, "apply_rope_cached: shape");
    const size_t nq = n_q_heads ? (size_t)(n_q_heads - 1) * q_head_stride + head_dim : 0;
    const size_t nk = n_kv_heads ? (size_t)(n_kv_heads - 1) * k_head_stride + head_dim : 0;
    Stage s;
    float* dq = nq ? s.in(0, q, nq) : nullptr;
    float* dk = nk ? s.in(1, k, nk) : nullptr;
    if (s.run(s.rc ? s.rc
                   : anelm_apply_rope(dq, dk, n_q_heads, n_kv_heads, head_dim, q_head_stride,
                                      k_head_stride, rot_dim, pos, theta, cos_row, sin_row,
                                      ANELM_ROPE_INTERLEAVED, nullptr)))
        return s.rc;
    if (nq && s.out(q, dq, nq)) return s.rc;
    if (nk) return s.out(k, dk, nk);
    return ANELM_OK;
}

int anelm_cpu_softmax(float* x, int n) {
    ANELM_NONNULL(x);
    ANELM_REQUIRE(n > 0, "softmax: n %d", n);
    Stage s;
    float* dx = s.in(0, x, (size_t)n);
    if (s.run(dx ? anelm_softmax(dx, n, 1, nullptr) : s.rc)) return s.rc;
    return s.out(x, dx, (size_t)n);
}

int anelm_cpu_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(W);
    ANELM_NONNULL(x);
    ANELM_REQUIRE(out_dim >= 0 && in_dim > 0, "matvec: %d x %d", out_dim, in_dim);
    Stage s;
    float* dW = s.in(0, W, (size_t)out_dim * in_dim);
    float* dx = s.in(1, x, (size_t)in_dim);
    float* dy = s.in<float>(2, nullptr, (size_t)out_dim);
    if (s.run(dy ? anelm_matvec(dy, dW, dx, out_dim, in_dim, nullptr) : s.rc)) return s.rc;
    return s.out(y, dy, (size_t)out_dim);
}

int anelm_cpu_l2_normalize(float* x, int dim) {
    ANELM_NONNULL(x);
    ANELM_REQUIRE(dim > 0, "l2_normalize: dim %d", dim);
    Stage s;
    float* dx = s.in(0, x, (size_t)dim);
    if (s.run(dx ? anelm_l2_normalize(dx, dim, 1, nullptr) : s.rc)) return s.rc;
    return s.out(x, dx, (size_t)dim);
}

int anelm_cpu_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                            const float* w, int channels, int kernel_size) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(conv_state);
    ANELM_NONNULL(state_pos);
    ANELM_NONNULL(x);
    ANELM_NONNULL(w);
    ANELM_REQUIRE(channels > 0 && kernel_size >= 2, "conv1d_update: channels %d kernel %d",
                  channels, kernel_size);
    const size_t ns = (size_t)channels * (kernel_size - 1);
    Stage s;
    float* dst = s.in(0, conv_state, ns);
    float* dx = s.in(1, x, (size_t)channels);
    float* dw = s.in(2, w, (size_t)channels * kernel_size);
    float* dy = s.in<float>(3, nullptr, (size_t)channels);
    if (s.run(dy ? anelm_conv1d_update(dy, dst, state_pos, dx, dw, channels, kernel_size, nullptr)
                 : s.rc))
        return s.rc;
    if (s.out(y, dy, (size_t)channels)) return s.rc;
    return s.out(conv_state, dst, ns);
}

int anelm_cpu_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                       float decay, float beta, int key_dim, int value_dim) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_REQUIRE(key_dim > 0 && value_dim > 0, "ssm_step: %d x %d", key_dim, value_dim);
    const size_t ns = (size_t)key_dim * value_dim;
    Stage s;
    float* dS = s.in(0, state, ns);
    float* dq = s.in(1, q, (size_t)key_dim);
    float* dk = s.in(2, k, (size_t)key_dim);
    float* dv = s.in(3, v, (size_t)value_dim);
    float* dy = s.in<float>(4, nullptr, (size_t)value_dim);
    if (s.run(dy ? anelm_ssm_step(dy, dS, dq, dk, dv, decay, beta, key_dim, value_dim, 0, nullptr)
                 : s.rc))
        return s.rc;
    if (s.out(y, dy, (size_t)value_dim)) return s.rc;
    return s.out(state, dS, ns);
}

int anelm_cpu_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                            int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                            int cache_start, int cache_len, int cache_capacity) {
    ANELM_NONNULL(out);
    ANELM_REQUIRE(n_heads > 0 && head_dim > 0 && n_kv_heads > 0, "gqa_attention: shape");
    const size_t no = (size_t)n_heads * head_dim;
    Stage s;
    float* dout = s.in<float>(0, nullptr, no);
    if (cache_len <= 0) {
        if (s.run(dout ? anelm_gqa_attention(dout, nullptr, nullptr, nullptr, ANELM_F32, n_heads,
                                             n_kv_heads, head_dim, q_head_stride, cache_start,
                                             cache_len, cache_capacity, nullptr)
                       : s.rc))
            return s.rc;
        return s.out(out, dout, no);
    }
    ANELM_NONNULL(q);
    ANELM_NONNULL(k_cache);
    ANELM_NONNULL(v_cache);
    const size_t nq = (size_t)(n_heads - 1) * q_head_stride + head_dim;
    const size_t nc = (size_t)cache_capacity * n_kv_heads * head_dim;
    float* dq = s.in(1, q, nq);
    float* dk = s.in(2, k_cache, nc);
    float* dv = s.in(3, v_cache, nc);
    if (s.run(dv ? anelm_gqa_attention(dout, dq, dk, dv, ANELM_F32, n_heads, n_kv_heads, head_dim,
                                       q_head_stride, cache_start, cache_len, cache_capacity,
                                       nullptr)
                 : s.rc))
        return s.rc;
    return s.out(out, dout, no);
}

}  // extern "C"
