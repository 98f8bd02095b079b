// Gated DeltaNet: decode step for all value heads and sequence prefill
// (dk = dv = 128).
//
// Reference: models/llm/qwen3_5.cpp:879-908 calling ssm_step
// (core/cpu_ops.cpp:131-146).  The reference reads each 64 KiB head state five
// times and writes it twice across four BLAS calls; here a workgroup holds a
// slab of state columns in registers and reads and writes it exactly once:
//   Sk[j] = sum_i S[i][j] k[i];  delta[j] = v[j] - Sk[j]
//   S'[i][j] = decay S[i][j] + beta k[i] delta[j];  y[j] = sum_i S'[i][j] q[i]
// Column j depends only on column j, so slabs of a head are independent.  The
// gated RMSNorm epilogue needs a whole head's y, so that variant gives one
// workgroup the whole head instead of combining slabs across workgroups.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

constexpr int kDK = 128;
constexpr int kDV = 128;

struct DnParams {
    float* y;
    float* state;
    const float* q;
    const float* k;
    const float* v;
    const float* a;
    const float* b;
    const float* A;
    const float* dt_bias;
    const float* z;
    const float* norm_w;
    int Hk, Hv, flags;
};

// CB state columns per workgroup of NT threads: thread t owns column
// t % CB for rows [(t / CB) * RPT, +RPT).
template <int CB, int NT, bool GATED>
__global__ __launch_bounds__(NT) void deltanet_decode_kernel(const DnParams p) {
    constexpr int RC = NT / CB;       // row chunks
    constexpr int RPT = kDK / RC;     // rows per thread
    static_assert(!GATED || CB == kDV, "the gated epilogue needs the whole head");
    __shared__ float qs[kDK], ks[kDK];
    __shared__ float red_a[RC][CB];
    __shared__ float red[NT / 64];

    const int h = blockIdx.y;
    const int tid = threadIdx.x;
    const int c = tid % CB, rc = tid / CB;
    const int j = blockIdx.x * CB + c;
    const int kh = h / (p.Hv / p.Hk);

    // The state slab is requested first; the prologue below overlaps it.
    float* S = p.state + (size_t)h * kDK * kDV;
    float s[RPT];
#pragma unroll
    for (int r = 0; r < RPT; r++) s[r] = S[(size_t)(rc * RPT + r) * kDV + j];

    // q, k of the key head: optional l2 normalisation (cpu_ops.cpp:82-87) and
    // the 1/sqrt(dk) query scale (qwen3_5.cpp:879-887).
    float qv = 0.f, kv = 0.f;
    if (tid < kDK) {
        qv = p.q[(size_t)kh * kDK + tid];
        kv = p.k[(size_t)kh * kDK + tid];
    }
    if (p.flags & ANELM_DN_L2NORM) {
        const float sq = block_sum<NT>(qv * qv, red);
        const float sk = block_sum<NT>(kv * kv, red);
        qv = qv * (1.0f / sqrtf(sq + 1e-12f));
        kv = kv * (1.0f / sqrtf(sk + 1e-12f));
    }
    qv = qv * (1.0f / sqrtf((float)kDK));
    if (tid < kDK) { qs[tid] = qv; ks[tid] = kv; }

    // Gates (qwen3_5.cpp:896-898; cpu_ops.h:13-14).
    const float beta = 1.0f / (1.0f + expf(-p.b[h]));
    const float sp = logf(1.0f + expf(p.a[h] + p.dt_bias[h]));
    const float decay = expf(-p.A[h] * sp);
    const bool tf = (p.flags & ANELM_DN_ORDER_TRANSFORMERS) != 0;
    const float vj = p.v[(size_t)h * kDV + j];
    __syncthreads();

    float part = 0.f;
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        if (tf) s[r] = decay * s[r];
        part = fmaf(s[r], ks[rc * RPT + r], part);
    }
    red_a[rc][c] = part;
    __syncthreads();
    float sk = 0.f;
#pragma unroll
    for (int i = 0; i < RC; i++) sk += red_a[i][c];
    const float delta = tf ? (vj - sk) * beta : vj - sk;
    __syncthreads();

    float yp = 0.f;
#pragma unroll
    for (int r = 0; r < RPT; r++) {
        const int i = rc * RPT + r;
        const float n = tf ? fmaf(ks[i], delta, s[r]) : fmaf(beta * ks[i], delta, decay * s[r]);
        S[(size_t)i * kDV + j] = n;
        yp = fmaf(n, qs[i], yp);
    }
    red_a[rc][c] = yp;
    __syncthreads();
    float yj = 0.f;
#pragma unroll
    for (int i = 0; i < RC; i++) yj += red_a[i][c];

    if constexpr (!GATED) {
        if (rc == 0) p.y[(size_t)h * kDV + j] = yj;
    } else {
        // rmsnorm_gated (cpu_ops.cpp:32-38): rmsnorm(y, w, 1e-6) * sigmoid(z) * z
        const float ss = block_sum<NT>(rc == 0 ? yj * yj : 0.f, red);
        const float inv = 1.0f / sqrtf(ss / (float)kDV + 1e-6f);
        if (rc == 0) {
            const float zi = p.z[(size_t)h * kDV + j];
            float o = (yj * inv) * p.norm_w[j];
            o = o / (1.0f + expf(-zi));
            p.y[(size_t)h * kDV + j] = o * zi;
        }
    }
}

// ---------------------------------------------------------------- prefill
// Pre-pass: per (token, key head) l2-normalise q and k and scale q
// (qwen3_5.cpp:879-887); per (token, value head) beta and decay
// (qwen3_5.cpp:896-898).
__global__ __launch_bounds__(kDK) void dn_prep_kernel(float* qn, float* kn, float* beta, float* decay,
                                                      const float* q, const float* k, const float* a,
                                                      const float* b, const float* A,
                                                      const float* dt_bias, int Hk, int Hv, int flags) {
    __shared__ float red[kDK / 64];
    const int t = blockIdx.x, kh = blockIdx.y, i = threadIdx.x;
    const size_t off = ((size_t)t * Hk + kh) * kDK + i;
    float qv = q[off], kv = k[off];
    if (flags & ANELM_DN_L2NORM) {
        const float sq = block_sum<kDK>(qv * qv, red);
        const float sk = block_sum<kDK>(kv * kv, red);
        qv = qv * (1.0f / sqrtf(sq + 1e-12f));
        kv = kv * (1.0f / sqrtf(sk + 1e-12f));
    }
    qn[off] = qv * (1.0f / sqrtf((float)kDK));
    kn[off] = kv;
    const int group = Hv / Hk;
    if (i < group) {
        const int h = kh * group + i;
        const size_t g = (size_t)t * Hv + h;
        beta[g] = 1.0f / (1.0f + expf(-b[g]));
        const float sp = logf(1.0f + expf(a[g] + dt_bias[h]));
        decay[g] = expf(-A[h] * sp);
    }
}

constexpr int kScanCB = 32;                 // columns per scan workgroup
constexpr int kScanNT = 256;
constexpr int kScanRC = kScanNT / kScanCB;  // 8 row chunks
constexpr int kScanRPT = kDK / kScanRC;     // 16 rows per thread

// Sequential scan over tokens: a workgroup owns a 32-column slab of one
// head's state in registers for the whole sequence (one HBM read and write of
// the state per call); per token it reads q, k, v and the gates and writes y.
__global__ __launch_bounds__(kScanNT) void dn_scan_kernel(float* y, float* state, const float* qn,
                                                          const float* kn, const float* v,
                                                          const float* beta, const float* decay,
                                                          int S, int Hk, int Hv, int flags) {
    __shared__ float red_a[2][kScanRC][kScanCB];
    const int h = blockIdx.y, slab = blockIdx.x, tid = threadIdx.x;
    const int c = tid % kScanCB, rc = tid / kScanCB;
    const int j = slab * kScanCB + c;
    const int kh = h / (Hv / Hk);
    const bool tf = (flags & ANELM_DN_ORDER_TRANSFORMERS) != 0;
    float* Sp = state + (size_t)h * kDK * kDV;
    float s[kScanRPT];
#pragma unroll
    for (int r = 0; r < kScanRPT; r++) s[r] = Sp[(size_t)(rc * kScanRPT + r) * kDV + j];
    for (int t = 0; t < S; t++) {
        const float* kt = kn + ((size_t)t * Hk + kh) * kDK + rc * kScanRPT;
        const float* qt = qn + ((size_t)t * Hk + kh) * kDK + rc * kScanRPT;
        float kr[kScanRPT], qr[kScanRPT];
#pragma unroll
        for (int r = 0; r < kScanRPT; r += 4) {
            const float4 k4 = *reinterpret_cast<const float4*>(kt + r);
            const float4 q4 = *reinterpret_cast<const float4*>(qt + r);
            kr[r] = k4.x; kr[r + 1] = k4.y; kr[r + 2] = k4.z; kr[r + 3] = k4.w;
            qr[r] = q4.x; qr[r + 1] = q4.y; qr[r + 2] = q4.z; qr[r + 3] = q4.w;
        }
        const float bt = beta[(size_t)t * Hv + h], dc = decay[(size_t)t * Hv + h];
        const float vj = v[((size_t)t * Hv + h) * kDV + j];
        const int buf = t & 1;
        float part = 0.f;
#pragma unroll
        for (int r = 0; r < kScanRPT; r++) {
            if (tf) s[r] = dc * s[r];
            part = fmaf(s[r], kr[r], part);
        }
        red_a[buf][rc][c] = part;
        __syncthreads();
        float sk = 0.f;
#pragma unroll
        for (int i = 0; i < kScanRC; i++) sk += red_a[buf][i][c];
        const float delta = tf ? (vj - sk) * bt : vj - sk;
        float yp = 0.f;
#pragma unroll
        for (int r = 0; r < kScanRPT; r++) {
            s[r] = tf ? fmaf(kr[r], delta, s[r]) : fmaf(bt * kr[r], delta, dc * s[r]);
            yp = fmaf(s[r], qr[r], yp);
        }
        __syncthreads();
        red_a[buf][rc][c] = yp;
        __syncthreads();
        if (rc == 0) {
            float yj = 0.f;
#pragma unroll
            for (int i = 0; i < kScanRC; i++) yj += red_a[buf][i][c];
            y[((size_t)t * Hv + h) * kDV + j] = yj;
        }
    }
#pragma unroll
    for (int r = 0; r < kScanRPT; r++) Sp[(size_t)(rc * kScanRPT + r) * kDV + j] = s[r];
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_deltanet_decode(float* y, float* state, const float* q, const float* k,
                                     const float* v, const float* a, const float* b,
                                     const float* A, const float* dt_bias, const float* z,
                                     const float* norm_w, int Hk, int Hv, int dk, int dv,
                                     int flags, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_NONNULL(q);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_NONNULL(a);
    ANELM_NONNULL(b);
    ANELM_NONNULL(A);
    ANELM_NONNULL(dt_bias);
    ANELM_REQUIRE(dk == kDK && dv == kDV, "deltanet_decode: dk=%d dv=%d (only 128x128)", dk, dv);
    ANELM_REQUIRE(Hk > 0 && Hv > 0 && Hv % Hk == 0, "deltanet_decode: Hv %d not a multiple of Hk %d",
                  Hv, Hk);
    ANELM_REQUIRE((flags & ~7) == 0, "deltanet_decode: unknown flags 0x%x", flags);
    hipStream_t st = as_stream(stream);
    DnParams p{};
    p.y = y;
    p.state = state;
    p.q = q;
    p.k = k;
    p.v = v;
    p.a = a;
    p.b = b;
    p.A = A;
    p.dt_bias = dt_bias;
    p.Hk = Hk;
    p.Hv = Hv;
    p.flags = flags;
    if (flags & ANELM_DN_GATED_NORM) {
        ANELM_NONNULL(z);
        ANELM_NONNULL(norm_w);
        p.z = z;
        p.norm_w = norm_w;
        hipLaunchKernelGGL((deltanet_decode_kernel<128, 512, true>), dim3(1, Hv), dim3(512), 0, st, p);
    } else {
        hipLaunchKernelGGL((deltanet_decode_kernel<32, 256, false>), dim3(kDV / 32, Hv), dim3(256), 0,
                           st, p);
    }
    ANELM_LAUNCHED("deltanet_decode_kernel");
    return ANELM_OK;
}

extern "C" int anelm_deltanet_prefill(float* y, float* state, const float* q, const float* k,
                                      const float* v, const float* a, const float* b,
                                      const float* A, const float* dt_bias, int S, int Hk, int Hv,
                                      int dk, int dv, int chunk, int flags, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_NONNULL(q);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_NONNULL(a);
    ANELM_NONNULL(b);
    ANELM_NONNULL(A);
    ANELM_NONNULL(dt_bias);
    ANELM_REQUIRE(dk == kDK && dv == kDV, "deltanet_prefill: dk=%d dv=%d (only 128x128)", dk, dv);
    ANELM_REQUIRE(Hk > 0 && Hv > 0 && Hv % Hk == 0 && Hv / Hk <= kDK,
                  "deltanet_prefill: Hv %d not a multiple of Hk %d", Hv, Hk);
    ANELM_REQUIRE(S >= 0, "deltanet_prefill: S %d", S);
    ANELM_REQUIRE(chunk > 0, "deltanet_prefill: chunk %d", chunk);
    ANELM_REQUIRE((flags & ~3) == 0, "deltanet_prefill: flags 0x%x (GATED_NORM is decode-only)", flags);
    if (S == 0) return ANELM_OK;
    hipStream_t st = as_stream(stream);
    const size_t nqk = (size_t)S * Hk * kDK, ng = (size_t)S * Hv;
    float* ws = static_cast<float*>(workspace((2 * nqk + 2 * ng) * sizeof(float), st));
    if (!ws) return ANELM_ENOMEM;
    float* qn = ws;
    float* kn = qn + nqk;
    float* beta = kn + nqk;
    float* decay = beta + ng;
    hipLaunchKernelGGL(dn_prep_kernel, dim3(S, Hk), dim3(kDK), 0, st, qn, kn, beta, decay, q, k, a, b,
                       A, dt_bias, Hk, Hv, flags);
    ANELM_LAUNCHED("dn_prep_kernel");
    hipLaunchKernelGGL(dn_scan_kernel, dim3(kDV / kScanCB, Hv), dim3(kScanNT), 0, st, y, state, qn,
                       kn, v, beta, decay, S, Hk, Hv, flags);
    ANELM_LAUNCHED("dn_scan_kernel");
    return ANELM_OK;
}
