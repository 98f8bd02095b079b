// Row-wise cpu_ops kernels: RMSNorm, gated RMSNorm, l2 normalisation, RoPE,
// SiLU, sigmoid gate, softmax, fp32 matvec, causal conv1d update and the
// single-head DeltaNet step.  Each follows the reference function named in
// include/anelm.h; one workgroup handles one row.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

constexpr int kNT = 256;

// core/cpu_ops.cpp:24-30
__global__ __launch_bounds__(kNT) void rmsnorm_kernel(float* out, const float* x, const float* w,
                                                      int dim, int xs, int os, float eps) {
    __shared__ float red[kNT / 64];
    const float* xr = x + (size_t)blockIdx.x * xs;
    float* orow = out + (size_t)blockIdx.x * os;
    constexpr int kReg = 16;   // rows up to 16 * kNT elements stay in registers
    if (dim <= kReg * kNT) {
        // every load of the row issued at once (one memory round trip), then
        // the sum and the scaled row from registers
        float v[kReg], wv[kReg];
#pragma unroll
        for (int k = 0; k < kReg; k++) {
            const int i = threadIdx.x + kNT * k;
            v[k] = i < dim ? xr[i] : 0.f;
            wv[k] = i < dim ? w[i] : 0.f;
        }
        float ss = 0.f;
#pragma unroll
        for (int k = 0; k < kReg; k++) ss += v[k] * v[k];
        ss = block_sum<kNT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
#pragma unroll
        for (int k = 0; k < kReg; k++) {
            const int i = threadIdx.x + kNT * k;
            if (i < dim) orow[i] = (v[k] * inv) * wv[k];
        }
        return;
    }
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kNT) ss += xr[i] * xr[i];
    ss = block_sum<kNT>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = threadIdx.x; i < dim; i += kNT) orow[i] = (xr[i] * inv) * w[i];
}

// core/cpu_ops.cpp:32-38
__global__ __launch_bounds__(kNT) void rmsnorm_gated_kernel(float* out, const float* x,
                                                            const float* z, const float* w, int dim) {
    __shared__ float red[kNT / 64];
    const size_t off = (size_t)blockIdx.x * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kNT) ss += x[off + i] * x[off + i];
    ss = block_sum<kNT>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)dim + 1e-6f);
    for (int i = threadIdx.x; i < dim; i += kNT) {
        const float zi = z[off + i];
        float o = (x[off + i] * inv) * w[i];
        o = o / (1.0f + expf(-zi));
        out[off + i] = o * zi;
    }
}

// The same for rows of at most 64 * PER elements: one wave per row, four
// rows per workgroup, the row held in registers and its sum of squares
// reduced inside the wave (no workgroup barrier).
template <int PER>
__global__ __launch_bounds__(kNT) void rmsnorm_gated_rows_kernel(float* out, const float* x, const float* z,
                                                                 const float* w, int dim, int n_rows) {
    const int row = blockIdx.x * (kNT / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n_rows) return;   // the whole wave leaves together
    const size_t off = (size_t)row * dim;
    float xv[PER], zv[PER];
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int i = lane + 64 * e;
        xv[e] = i < dim ? x[off + i] : 0.f;
        zv[e] = i < dim ? z[off + i] : 0.f;
        ss += xv[e] * xv[e];
    }
    ss = wave_sum(ss);
    const float inv = 1.0f / sqrtf(ss / (float)dim + 1e-6f);
#pragma unroll
    for (int e = 0; e < PER; e++) {
        const int i = lane + 64 * e;
        if (i < dim) {
            float o = (xv[e] * inv) * w[i];
            o = o / (1.0f + expf(-zv[e]));
            out[off + i] = o * zv[e];
        }
    }
}

// The 128-element rows of a DeltaNet head (8-byte aligned): lane l holds
// elements 2l, 2l + 1, one 8-byte load per operand.
__global__ __launch_bounds__(kNT) void rmsnorm_gated_rows128_kernel(float* out, const float* x, const float* z,
                                                                    const float* w, int n_rows) {
    const int row = blockIdx.x * (kNT / 64) + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= n_rows) return;   // the whole wave leaves together
    const size_t off = (size_t)row * 128 + 2 * lane;
    const float2 xv = *reinterpret_cast<const float2*>(x + off);
    const float2 zv = *reinterpret_cast<const float2*>(z + off);
    const float2 wv = *reinterpret_cast<const float2*>(w + 2 * lane);
    const float ss = wave_sum(xv.x * xv.x + xv.y * xv.y);
    const float inv = 1.0f / sqrtf(ss / 128.0f + 1e-6f);
    float o0 = (xv.x * inv) * wv.x, o1 = (xv.y * inv) * wv.y;
    o0 = o0 / (1.0f + expf(-zv.x));
    o1 = o1 / (1.0f + expf(-zv.y));
    *reinterpret_cast<float2*>(out + off) = make_float2(o0 * zv.x, o1 * zv.y);
}

// core/cpu_ops.cpp:82-87
__global__ __launch_bounds__(kNT) void l2norm_kernel(float* x, int dim) {
    __shared__ float red[kNT / 64];
    float* r = x + (size_t)blockIdx.x * dim;
    float ss = 0.f;
    for (int i = threadIdx.x; i < dim; i += kNT) ss += r[i] * r[i];
    ss = block_sum<kNT>(ss, red);
    const float inv = 1.0f / sqrtf(ss + 1e-12f);
    for (int i = threadIdx.x; i < dim; i += kNT) r[i] = r[i] * inv;
}

struct RopeArgs {
    float* q;
    float* k;
    int nq, nkv, qs, ks, pairs, mode;
    float cs[kMaxRotPairs];
    float sn[kMaxRotPairs];
};

// core/cpu_ops.cpp:40-63; one thread per (head, pair)
__global__ void rope_kernel(const RopeArgs a) {
    const int idx = blockIdx.x * blockDim.x + threadIdx.x;
    const int total = (a.nq + a.nkv) * a.pairs;
    if (idx >= total) return;
    const int h = idx / a.pairs, j = idx % a.pairs;
    float* v = (h < a.nq) ? a.q + (size_t)h * a.qs : a.k + (size_t)(h - a.nq) * a.ks;
    const int i0 = a.mode == 0 ? 2 * j : j;
    const int i1 = a.mode == 0 ? 2 * j + 1 : j + a.pairs;
    const float* cs = a.cs;   // pointer into the argument segment (see attn_decode.hip)
    const float* sn = a.sn;
    const float c = cs[j], s = sn[j];
    const float v0 = v[i0], v1 = v[i1];
    rotate_pair(v[i0], v[i1], v0, v1, c, s);
}

// core/cpu_ops.cpp:6-13 and :15-22
__global__ void silu_kernel(float* x, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = x[i] / (expf(-x[i]) + 1.0f);
}
__global__ void mul_sigmoid_kernel(float* y, const float* z, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = y[i] / (expf(-z[i]) + 1.0f);
}

// core/cpu_ops.cpp:65-75
__global__ __launch_bounds__(kNT) void softmax_kernel(float* x, int n) {
    __shared__ float red[kNT / 64];
    float* r = x + (size_t)blockIdx.x * n;
    float m = -INFINITY;
    for (int i = threadIdx.x; i < n; i += kNT) m = fmaxf(m, r[i]);
    m = block_max<kNT>(m, red);
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += kNT) {
        const float e = expf(r[i] - m);
        r[i] = e;
        s += e;
    }
    s = block_sum<kNT>(s, red);
    const float inv = 1.0f / s;
    for (int i = threadIdx.x; i < n; i += kNT) r[i] = r[i] * inv;
}

// core/cpu_ops.cpp:77-80; one wave per output row
__global__ __launch_bounds__(kNT) void matvec_kernel(float* y, const float* W, const float* x,
                                                     int out_dim, int in_dim) {
    const int row = blockIdx.x * (kNT / 64) + (threadIdx.x >> 6);
    if (row >= out_dim) return;
    const int lane = threadIdx.x & 63;
    const float* wr = W + (size_t)row * in_dim;
    float s = 0.f;
    for (int c = lane; c < in_dim; c += 64) s = fmaf(wr[c], x[c], s);
    s = wave_sum(s);
    if (lane == 0) y[row] = s;
}

// core/cpu_ops.cpp:89-129; one thread per channel
__global__ void conv1d_kernel(float* y, float* st, const float* x, const float* w, int channels,
                              int ks, int pos) {
    const int c = blockIdx.x * blockDim.x + threadIdx.x;
    if (c >= channels) return;
    const int sl = ks - 1;
    float sum = 0.f;
    for (int j = 0; j < sl; j++) {
        int idx = pos + j;
        if (idx >= sl) idx -= sl;
        sum += st[(size_t)c * sl + idx] * w[(size_t)c * ks + j];
    }
    const float xc = x[c];
    y[c] = sum + xc * w[(size_t)c * ks + sl];
    st[(size_t)c * sl + pos] = xc;
}

// core/cpu_ops.cpp:131-146 for one head; one thread per value column j keeps
// its column of the state in registers between the two passes when it fits
// (key_dim <= 128); a 256-long column would spill to scratch, so it is read
// again (from cache) in the second pass instead.
template <int DK>
__global__ __launch_bounds__(kNT) void ssm_step_kernel(float* y, float* S, const float* q,
                                                       const float* k, const float* v, float decay,
                                                       float beta, int dv, int order) {
    constexpr bool kHold = DK <= 128;
    constexpr int kUnroll = kHold ? DK : 16;   // a fully unrolled re-read would reuse the first loads
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= dv) return;
    float col[kHold ? DK : 1];
    float sk = 0.f;
#pragma unroll kUnroll
    for (int i = 0; i < DK; i++) {
        float s = S[(size_t)i * dv + j];
        if (order) s = decay * s;
        if constexpr (kHold) col[i] = s;
        sk = fmaf(s, k[i], sk);
    }
    const float delta = order ? (v[j] - sk) * beta : v[j] - sk;
    float yo = 0.f;
#pragma unroll kUnroll
    for (int i = 0; i < DK; i++) {
        float c;
        if constexpr (kHold) {
            c = col[i];
        } else {
            c = S[(size_t)i * dv + j];
            if (order) c = decay * c;
        }
        float s = order ? fmaf(k[i], delta, c) : fmaf(beta * k[i], delta, decay * c);
        S[(size_t)i * dv + j] = s;
        yo = fmaf(s, q[i], yo);
    }
    y[j] = yo;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" {

int anelm_rmsnorm(float* out, const float* x, const float* weight, int dim, int n_rows,
                  int x_stride, int out_stride, float eps, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(x);
    ANELM_NONNULL(weight);
    ANELM_REQUIRE(dim > 0 && n_rows >= 0 && x_stride >= dim && out_stride >= dim,
                  "rmsnorm: dim %d rows %d strides %d/%d", dim, n_rows, x_stride, out_stride);
    if (n_rows == 0) return ANELM_OK;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3(n_rows), dim3(kNT), 0, as_stream(stream), out, x,
                       weight, dim, x_stride, out_stride, eps);
    ANELM_LAUNCHED("rmsnorm_kernel");
    return ANELM_OK;
}

int anelm_rmsnorm_gated(float* out, const float* x, const float* z, const float* weight, int dim,
                        int n_rows, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(x);
    ANELM_NONNULL(z);
    ANELM_NONNULL(weight);
    ANELM_REQUIRE(dim > 0 && n_rows >= 0, "rmsnorm_gated: dim %d rows %d", dim, n_rows);
    if (n_rows == 0) return ANELM_OK;
    hipStream_t st = as_stream(stream);
    const dim3 rgrid((unsigned)((n_rows + kNT / 64 - 1) / (kNT / 64)));
    const bool al8 = ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(x) |
                       reinterpret_cast<uintptr_t>(z) | reinterpret_cast<uintptr_t>(weight)) & 7) == 0;
    if (dim == 128 && al8) {
        hipLaunchKernelGGL(rmsnorm_gated_rows128_kernel, rgrid, dim3(kNT), 0, st, out, x, z, weight, n_rows);
        ANELM_LAUNCHED("rmsnorm_gated_rows128_kernel");
    } else if (dim <= 128) {
        hipLaunchKernelGGL(rmsnorm_gated_rows_kernel<2>, rgrid, dim3(kNT), 0, st, out, x, z, weight, dim, n_rows);
        ANELM_LAUNCHED("rmsnorm_gated_rows_kernel");
    } else if (dim <= 256) {
        hipLaunchKernelGGL(rmsnorm_gated_rows_kernel<4>, rgrid, dim3(kNT), 0, st, out, x, z, weight, dim, n_rows);
        ANELM_LAUNCHED("rmsnorm_gated_rows_kernel");
    } else {
        hipLaunchKernelGGL(rmsnorm_gated_kernel, dim3(n_rows), dim3(kNT), 0, st, out, x, z, weight, dim);
        ANELM_LAUNCHED("rmsnorm_gated_kernel");
    }
    return ANELM_OK;
}

int anelm_l2_normalize(float* x, int dim, int n_rows, void* stream) {
    ANELM_NONNULL(x);
    ANELM_REQUIRE(dim > 0 && n_rows >= 0, "l2_normalize: dim %d rows %d", dim, n_rows);
    if (n_rows == 0) return ANELM_OK;
    hipLaunchKernelGGL(l2norm_kernel, dim3(n_rows), dim3(kNT), 0, as_stream(stream), x, dim);
    ANELM_LAUNCHED("l2norm_kernel");
    return ANELM_OK;
}

int anelm_apply_rope(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                     int q_head_stride, int k_head_stride, int rot_dim, int pos, float theta,
                     const float* cos_row, const float* sin_row, int rope_mode, void* stream) {
    ANELM_REQUIRE(n_q_heads >= 0 && n_kv_heads >= 0, "rope: negative head count");
    ANELM_REQUIRE(n_q_heads == 0 || q != nullptr, "rope: q is NULL");
    ANELM_REQUIRE(n_kv_heads == 0 || k != nullptr, "rope: k is NULL");
    ANELM_REQUIRE(rot_dim >= 0 && rot_dim % 2 == 0 && rot_dim <= head_dim &&
                      rot_dim / 2 <= kMaxRotPairs,
                  "rope: rot_dim %d must be even, <= head_dim %d and <= 256", rot_dim, head_dim);
    ANELM_REQUIRE(rope_mode == ANELM_ROPE_INTERLEAVED || rope_mode == ANELM_ROPE_HALF_SPLIT,
                  "rope: mode %d unknown", rope_mode);
    RopeArgs a{};
    a.q = q;
    a.k = k;
    a.nq = n_q_heads;
    a.nkv = n_kv_heads;
    a.qs = q_head_stride;
    a.ks = k_head_stride;
    a.pairs = rot_dim / 2;
    a.mode = rope_mode;
    if (cos_row && sin_row) {
        for (int j = 0; j < a.pairs; j++) { a.cs[j] = cos_row[j]; a.sn[j] = sin_row[j]; }
    } else {
        rope_row(a.cs, a.sn, rot_dim, pos, theta);
    }
    const int total = (n_q_heads + n_kv_heads) * a.pairs;
    if (total == 0) return ANELM_OK;
    hipLaunchKernelGGL(rope_kernel, dim3((total + 255) / 256), dim3(256), 0, as_stream(stream), a);
    ANELM_LAUNCHED("rope_kernel");
    return ANELM_OK;
}

int anelm_silu_inplace(float* x, int n, void* stream) {
    ANELM_NONNULL(x);
    ANELM_REQUIRE(n >= 0, "silu: n %d", n);
    if (n == 0) return ANELM_OK;
    hipLaunchKernelGGL(silu_kernel, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream), x, n);
    ANELM_LAUNCHED("silu_kernel");
    return ANELM_OK;
}

int anelm_mul_sigmoid_inplace(float* y, const float* z, int n, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(z);
    ANELM_REQUIRE(n >= 0, "mul_sigmoid: n %d", n);
    if (n == 0) return ANELM_OK;
    hipLaunchKernelGGL(mul_sigmoid_kernel, dim3((n + 255) / 256), dim3(256), 0, as_stream(stream),
                       y, z, n);
    ANELM_LAUNCHED("mul_sigmoid_kernel");
    return ANELM_OK;
}

int anelm_softmax(float* x, int n, int n_rows, void* stream) {
    ANELM_NONNULL(x);
    ANELM_REQUIRE(n > 0 && n_rows >= 0, "softmax: n %d rows %d", n, n_rows);
    if (n_rows == 0) return ANELM_OK;
    hipLaunchKernelGGL(softmax_kernel, dim3(n_rows), dim3(kNT), 0, as_stream(stream), x, n);
    ANELM_LAUNCHED("softmax_kernel");
    return ANELM_OK;
}

int anelm_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(W);
    ANELM_NONNULL(x);
    ANELM_REQUIRE(out_dim >= 0 && in_dim > 0, "matvec: %d x %d", out_dim, in_dim);
    if (out_dim == 0) return ANELM_OK;
    const int rows_per_block = kNT / 64;
    hipLaunchKernelGGL(matvec_kernel, dim3((out_dim + rows_per_block - 1) / rows_per_block),
                       dim3(kNT), 0, as_stream(stream), y, W, x, out_dim, in_dim);
    ANELM_LAUNCHED("matvec_kernel");
    return ANELM_OK;
}

int anelm_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                        const float* w, int channels, int kernel_size, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(conv_state);
    ANELM_NONNULL(state_pos);
    ANELM_NONNULL(x);
    ANELM_NONNULL(w);
    ANELM_REQUIRE(channels > 0 && kernel_size >= 2, "conv1d: channels %d kernel %d", channels,
                  kernel_size);
    ANELM_REQUIRE(*state_pos >= 0 && *state_pos < kernel_size - 1, "conv1d: state_pos %d",
                  *state_pos);
    hipLaunchKernelGGL(conv1d_kernel, dim3((channels + 255) / 256), dim3(256), 0,
                       as_stream(stream), y, conv_state, x, w, channels, kernel_size, *state_pos);
    ANELM_LAUNCHED("conv1d_kernel");
    int pos = *state_pos + 1;
    if (pos == kernel_size - 1) pos = 0;
    *state_pos = pos;
    return ANELM_OK;
}

int anelm_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                   float decay, float beta, int key_dim, int value_dim, int flags, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_NONNULL(q);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_REQUIRE(value_dim > 0, "ssm_step: value_dim %d", value_dim);
    const int order = (flags & ANELM_DN_ORDER_TRANSFORMERS) ? 1 : 0;
    dim3 grid((value_dim + kNT - 1) / kNT), block(kNT);
    hipStream_t st = as_stream(stream);
    switch (key_dim) {
        case 64: hipLaunchKernelGGL(ssm_step_kernel<64>, grid, block, 0, st, y, state, q, k, v, decay, beta, value_dim, order); break;
        case 128: hipLaunchKernelGGL(ssm_step_kernel<128>, grid, block, 0, st, y, state, q, k, v, decay, beta, value_dim, order); break;
        case 256: hipLaunchKernelGGL(ssm_step_kernel<256>, grid, block, 0, st, y, state, q, k, v, decay, beta, value_dim, order); break;
        default: return set_error(ANELM_EINVAL, "ssm_step: key_dim %d unsupported (64,128,256)", key_dim);
    }
    ANELM_LAUNCHED("ssm_step_kernel");
    return ANELM_OK;
}

}  // extern "C"
