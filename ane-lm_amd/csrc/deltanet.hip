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
                                                      float* ldecay, const float* q, const float* k,
                                                      const float* a, const float* b, const float* A,
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
        if (ldecay) ldecay[g] = -A[h] * sp;   // log of the decay, for the chunked form
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

// ------------------------------------------------------- chunked prefill
// The recurrence over a chunk of C = 64 tokens in closed form (per value head,
// chunk start state S0, lg_t = sum_{j<=t} log g_j inside the chunk):
//   cpu_ops order (core/cpu_ops.cpp:131-146): u_t = beta_t (v_t - S_{t-1}^T k_t)
//     S_t = exp(lg_t) S0 + sum_{i<=t} exp(lg_t - lg_i) k_i u_i^T
//     u_t = beta_t (v_t - exp(lg_{t-1}) S0^T k_t) - sum_{i<t} A_ti u_i,
//     A_ti = beta_t exp(lg_{t-1} - lg_i) (k_t . k_i)
//   decay-first order: the same with lg_{t-1} replaced by lg_t in A and u.
// With T = (I + A)^-1 (unit lower triangular):
//   Ut = T diag(beta) V,  Wm = T diag(beta exp(lg_{t-1 or t})) K,  U = Ut - Wm S0
//   y  = Op + Qh S0,      Op = P Ut,  Qh = diag(exp(lg)) Q - P Wm,
//                         P_ti = exp(lg_t - lg_i) (q_t . k_i), i <= t
//   S_end = gC S0 + Kh^T U,  Kh = diag(exp(lg_L - lg)) K,  gC = exp(lg_L)
// Everything but the three products with S0 is independent of the state and
// is computed for all chunks at once (dn_chunk_pre_kernel); dn_chunk_seq_kernel
// then carries the state through the chunks.  Decay ratios are formed in log
// space (all exponents <= 0).  Rows past the sequence end are zero (beta 0,
// log decay 0), so they change nothing.
constexpr int kChunk = 64;
constexpr int kCMat = kChunk * kDK;             // floats per chunk matrix
constexpr int kCRec = 5 * kCMat + 64;           // Ut, Wm, Op, Qh, Kh, gC
constexpr int kPreNT = 256;
constexpr int kTS = kChunk + 4;                 // row stride of the transposed tiles

template <bool TF>
__global__ __launch_bounds__(kPreNT, 2) void dn_chunk_pre_kernel(float* __restrict__ rec, const float* __restrict__ qn,
                                                                  const float* __restrict__ kn,
                                                                  const float* __restrict__ v,
                                                                  const float* __restrict__ beta,
                                                                  const float* __restrict__ ldecay, int S, int Hk,
                                                                  int Hv) {
    // K^T and Q^T tiles ([d][t]) for the dot products; afterwards the same
    // space holds A and P ([t][i]), so two workgroups fit on a CU
    __shared__ __attribute__((aligned(16))) float T0[kDK][kTS];
    __shared__ __attribute__((aligned(16))) float T1[kDK][kTS];
    __shared__ float lg[kChunk + 1];                                // lg[t + 1]; lg[0] = 0
    __shared__ float bt[kChunk];
    float (*KT)[kTS] = T0;
    float (*QT)[kTS] = T1;
    float (*Am)[kTS] = T0;   // rows 0..63 of T0, after the dot products
    float (*Pm)[kTS] = T1;
    const int c = blockIdx.x, h = blockIdx.y, tid = threadIdx.x;
    const int kh = h / (Hv / Hk);
    const int t0 = c * kChunk, L = min(kChunk, S - t0);
    {
        // all 64 loads of this thread in flight together, then the transposed stores
        constexpr int NE = kCMat / kPreNT;
        float kv[NE], qv[NE];
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int e = tid + kPreNT * k, t = e / kDK, d = e - t * kDK;
            const size_t off = ((size_t)(t0 + min(t, L - 1)) * Hk + kh) * kDK + d;
            kv[k] = kn[off];
            qv[k] = qn[off];
        }
#pragma unroll
        for (int k = 0; k < NE; k++) {
            const int e = tid + kPreNT * k, t = e / kDK, d = e - t * kDK;
            KT[d][t] = t < L ? kv[k] : 0.f;
            QT[d][t] = t < L ? qv[k] : 0.f;
        }
    }
    if (tid < kChunk) bt[tid] = tid < L ? beta[(size_t)(t0 + tid) * Hv + h] : 0.f;
    if (tid == 0) {
        float acc = 0.f;
        lg[0] = 0.f;
        for (int t = 0; t < kChunk; t++) {
            if (t < L) acc += ldecay[(size_t)(t0 + t) * Hv + h];
            lg[t + 1] = acc;
        }
    }
    __syncthreads();
    // k_t . k_i and q_t . k_i for 4x4 blocks with i <= t
    const int tb = tid >> 4, ib = tid & 15;
    float kk[4][4], qk[4][4];
#pragma unroll
    for (int x = 0; x < 4; x++)
#pragma unroll
        for (int y = 0; y < 4; y++) kk[x][y] = qk[x][y] = 0.f;
    if (ib <= tb) {
#pragma unroll 4
        for (int d = 0; d < kDK; d++) {
            const float4 kt = *reinterpret_cast<const float4*>(&KT[d][4 * tb]);
            const float4 ki = *reinterpret_cast<const float4*>(&KT[d][4 * ib]);
            const float4 qt = *reinterpret_cast<const float4*>(&QT[d][4 * tb]);
            const float a4[4] = {kt.x, kt.y, kt.z, kt.w}, b4[4] = {ki.x, ki.y, ki.z, ki.w};
            const float q4[4] = {qt.x, qt.y, qt.z, qt.w};
#pragma unroll
            for (int x = 0; x < 4; x++)
#pragma unroll
                for (int y = 0; y < 4; y++) {
                    kk[x][y] = fmaf(a4[x], b4[y], kk[x][y]);
                    qk[x][y] = fmaf(q4[x], b4[y], qk[x][y]);
                }
        }
    }
    __syncthreads();   // the tiles are overwritten by A and P below
#pragma unroll
    for (int x = 0; x < 4; x++) {
        const int t = 4 * tb + x;
        const float lgT = TF ? lg[t + 1] : lg[t];
#pragma unroll
        for (int y = 0; y < 4; y++) {
            const int i = 4 * ib + y;
            Am[t][i] = i < t ? bt[t] * expf(lgT - lg[i + 1]) * kk[x][y] : 0.f;
            Pm[t][i] = i <= t ? expf(lg[t + 1] - lg[i + 1]) * qk[x][y] : 0.f;
        }
    }
    __syncthreads();
    // thread j < 128: column j of Ut (right-hand side beta V), then Op = P Ut;
    // thread j >= 128: column j-128 of Wm (beta exp(lg) K), then Qh = exp(lg) Q - P Wm
    const int j = tid & (kDK - 1);
    const bool wpart = tid >= kDK;
    float* out = rec + ((size_t)c * Hv + h) * kCRec;
    const float* src = wpart ? kn : v;
    float u[kChunk];
    // right-hand sides first (all global loads in flight together), then the
    // forward substitution in place
#pragma unroll
    for (int t = 0; t < kChunk; t++) {
        const size_t off = wpart ? ((size_t)(t0 + min(t, L - 1)) * Hk + kh) * kDK + j
                                 : ((size_t)(t0 + min(t, L - 1)) * Hv + h) * kDV + j;
        u[t] = src[off];
    }
#pragma unroll
    for (int t = 0; t < kChunk; t++) {
        const float scale = t < L ? bt[t] * (wpart ? expf(TF ? lg[t + 1] : lg[t]) : 1.0f) : 0.f;
        // four partial sums (shorter dependency chains); A row t read as
        // float4s (same address in every lane: LDS broadcast)
        float b0 = u[t] * scale, b1 = 0.f, b2 = 0.f, b3 = 0.f;
#pragma unroll
        for (int i4 = 0; i4 < t; i4 += 4) {
            const float4 a4 = *reinterpret_cast<const float4*>(&Am[t][i4]);
            b0 = fmaf(-a4.x, u[i4], b0);
            if (i4 + 1 < t) b1 = fmaf(-a4.y, u[i4 + 1], b1);
            if (i4 + 2 < t) b2 = fmaf(-a4.z, u[i4 + 2], b2);
            if (i4 + 3 < t) b3 = fmaf(-a4.w, u[i4 + 3], b3);
        }
        u[t] = (b0 + b1) + (b2 + b3);
        // row t is finished here (the data dependency keeps its arithmetic
        // before this point) and the next rows' loads stay after it
        asm volatile("" : "+v"(u[t]) :: "memory");
    }
    float* mu = out + (wpart ? kCMat : 0);              // Ut or Wm
    float* mr = out + (wpart ? 3 * kCMat : 2 * kCMat);  // Op or Qh
    float* kh_out = out + 4 * kCMat;
    const float lgL = lg[kChunk];
#pragma unroll
    for (int t = 0; t < kChunk; t++) {
        float r0 = 0.f, r1 = 0.f, r2 = 0.f, r3 = 0.f;
#pragma unroll
        for (int i4 = 0; i4 <= t; i4 += 4) {
            const float4 p4 = *reinterpret_cast<const float4*>(&Pm[t][i4]);
            r0 = fmaf(p4.x, u[i4], r0);
            if (i4 + 1 <= t) r1 = fmaf(p4.y, u[i4 + 1], r1);
            if (i4 + 2 <= t) r2 = fmaf(p4.z, u[i4 + 2], r2);
            if (i4 + 3 <= t) r3 = fmaf(p4.w, u[i4 + 3], r3);
        }
        float r = (r0 + r1) + (r2 + r3);
        mu[t * kDK + j] = u[t];
        if (wpart) {
            const size_t off = ((size_t)(t0 + min(t, L - 1)) * Hk + kh) * kDK + j;
            const float qv = t < L ? qn[off] : 0.f, kv = t < L ? kn[off] : 0.f;
            r = expf(lg[t + 1]) * qv - r;
            kh_out[t * kDK + j] = expf(lgL - lg[t + 1]) * kv;
        }
        mr[t * kDK + j] = r;
        asm volatile("" : "+v"(r) :: "memory");
    }
    if (tid == 0) out[5 * kCMat] = expf(lgL);
}

// Sequential part: workgroup (slab of 16 state columns, value head) keeps its
// 128 x 16 slab of S in registers across all chunks; thread (c = tid & 15,
// rb = tid >> 4) holds rows 8 rb .. 8 rb + 7 of column c.  Per chunk:
//   U = Ut - Wm S0;  y = Op + Qh S0;  S = gC S0 + Kh^T U
// with Wm, Qh, Kh staged through LDS (the next one is loaded into registers
// while the current one is used); the 16 row-block partial sums are first
// combined within each wave (4 row blocks per wave) and then across the 4
// waves in LDS.
constexpr int kSeqNT = 256;
constexpr int kSeqCB = 16;
constexpr int kSlabs = kDV / kSeqCB;
__device__ __forceinline__ void dn_seq_fetch(float4 (&r)[8], const float* src, int tid) {
#pragma unroll
    for (int k = 0; k < 8; k++) r[k] = reinterpret_cast<const float4*>(src)[tid + kSeqNT * k];
}
__device__ __forceinline__ void dn_seq_park(float* dst, const float4 (&r)[8], int tid) {
#pragma unroll
    for (int k = 0; k < 8; k++) reinterpret_cast<float4*>(dst)[tid + kSeqNT * k] = r[k];
}
// part[t] = sum over this thread's 8 rows of M[t][row] * s[row], summed over
// the wave's 4 row blocks (lanes sharing lane & 15)
__device__ __forceinline__ void dn_seq_rowdot(float (&part)[kChunk], const float* M, const float (&s)[8], int rb) {
#pragma unroll
    for (int t = 0; t < kChunk; t++) {
        const float4* mrow = reinterpret_cast<const float4*>(M + t * kDK + 8 * rb);
        const float4 m0 = mrow[0], m1 = mrow[1];
        const float a0 = fmaf(m0.y, s[1], m0.x * s[0]);
        const float a1 = fmaf(m0.w, s[3], m0.z * s[2]);
        const float a2 = fmaf(m1.y, s[5], m1.x * s[4]);
        const float a3 = fmaf(m1.w, s[7], m1.z * s[6]);
        part[t] = (a0 + a1) + (a2 + a3);
    }
#pragma unroll
    for (int t = 0; t < kChunk; t++) {
        part[t] += __shfl_xor(part[t], 16, 64);
        part[t] += __shfl_xor(part[t], 32, 64);
    }
}

__global__ __launch_bounds__(kSeqNT) void dn_chunk_seq_kernel(float* __restrict__ y, float* __restrict__ state,
                                                              const float* __restrict__ rec, int S, int Hv,
                                                              int n_chunks) {
    __shared__ __attribute__((aligned(16))) float M[2][kCMat];           // 64 KB: current / next matrix
    __shared__ __attribute__((aligned(16))) float red[4][kChunk][kSeqCB];  // 16 KB: per-wave sums
    __shared__ __attribute__((aligned(16))) float Ul[kChunk][kSeqCB];      // 4 KB
    // XCD-aware: workgroups are dealt round-robin over the 8 XCDs (id % 8);
    // the 8 slabs of a head share its chunk matrices, so they go to one XCD
    // (one L2) -- with Hv a multiple of 8, heads 4x .. 4x+3 on XCD x
    const int nwg = gridDim.x, id = blockIdx.x;
    const int per_xcd = nwg / 8, k = id / 8, xcd = id % 8;
    const int h = (xcd * per_xcd + k) / kSlabs, slab = (xcd * per_xcd + k) % kSlabs;
    const int tid = threadIdx.x;
    const int c = tid & (kSeqCB - 1), rb = tid >> 4, w = tid >> 6;
    const bool lead = (tid & 63) < kSeqCB;   // one lane per column of each wave
    const int col = slab * kSeqCB + c;
    float* Sp = state + (size_t)h * kDK * kDV;
    float s[8];
#pragma unroll
    for (int r = 0; r < 8; r++) s[r] = Sp[(size_t)(8 * rb + r) * kDV + col];
    float4 nxt[8];
    dn_seq_fetch(nxt, rec + (size_t)h * kCRec + kCMat, tid);   // Wm of chunk 0
    int buf = 0;
    for (int ch = 0; ch < n_chunks; ch++) {
        const float* rc = rec + ((size_t)ch * Hv + h) * kCRec;
        const int t0 = ch * kChunk, L = min(kChunk, S - t0);
        float part[kChunk];
        // this thread's 4 rows of Ut and Op (t = 4 rb + k), issued early
        float ut[4], op[4];
        const float gC = rc[5 * kCMat];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ut[k] = rc[(4 * rb + k) * kDK + col];
            op[k] = rc[2 * kCMat + (4 * rb + k) * kDK + col];
        }
        // ---- U = Ut - Wm S0
        dn_seq_park(M[buf], nxt, tid);
        lds_barrier();
        dn_seq_fetch(nxt, rc + 3 * kCMat, tid);                 // Qh
        dn_seq_rowdot(part, M[buf], s, rb);
        if (lead) {
#pragma unroll
            for (int t = 0; t < kChunk; t++) red[w][t][c] = part[t];
        }
        buf ^= 1;
        dn_seq_park(M[buf], nxt, tid);
        lds_barrier();
        dn_seq_fetch(nxt, rc + 4 * kCMat, tid);                 // Kh
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int t = 4 * rb + k;
            Ul[t][c] = ut[k] - (red[0][t][c] + red[1][t][c] + red[2][t][c] + red[3][t][c]);
        }
        // ---- y = Op + Qh S0
        dn_seq_rowdot(part, M[buf], s, rb);
        lds_barrier();   // red consumed by the U rows above
        if (lead) {
#pragma unroll
            for (int t = 0; t < kChunk; t++) red[w][t][c] = part[t];
        }
        buf ^= 1;
        dn_seq_park(M[buf], nxt, tid);
        lds_barrier();
        if (ch + 1 < n_chunks) dn_seq_fetch(nxt, rc + (size_t)Hv * kCRec + kCMat, tid);   // next Wm
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int t = 4 * rb + k;
            if (t < L)
                y[((size_t)(t0 + t) * Hv + h) * kDV + col] =
                    op[k] + (red[0][t][c] + red[1][t][c] + red[2][t][c] + red[3][t][c]);
        }
        // ---- S = gC S0 + Kh^T U
        const float* Kh = M[buf];
#pragma unroll
        for (int r = 0; r < 8; r++) s[r] *= gC;
#pragma unroll 4
        for (int t = 0; t < kChunk; t++) {
            const float uv = Ul[t][c];
            const float4* krow = reinterpret_cast<const float4*>(Kh + t * kDK + 8 * rb);
            const float4 k0 = krow[0], k1 = krow[1];
            s[0] = fmaf(k0.x, uv, s[0]); s[1] = fmaf(k0.y, uv, s[1]); s[2] = fmaf(k0.z, uv, s[2]); s[3] = fmaf(k0.w, uv, s[3]);
            s[4] = fmaf(k1.x, uv, s[4]); s[5] = fmaf(k1.y, uv, s[5]); s[6] = fmaf(k1.z, uv, s[6]); s[7] = fmaf(k1.w, uv, s[7]);
        }
        lds_barrier();   // Ul, red and M[buf] are rewritten in the next chunk
        buf ^= 1;
    }
#pragma unroll
    for (int r = 0; r < 8; r++) Sp[(size_t)(8 * rb + r) * kDV + col] = s[r];
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
    ANELM_REQUIRE(chunk == kChunk || chunk == 1,
                  "deltanet_prefill: chunk %d (64: chunked form; 1: token-by-token scan)", chunk);
    ANELM_REQUIRE((flags & ~3) == 0, "deltanet_prefill: flags 0x%x (GATED_NORM is decode-only)", flags);
    if (S == 0) return ANELM_OK;
    hipStream_t st = as_stream(stream);
    const size_t nqk = (size_t)S * Hk * kDK, ng = (size_t)S * Hv;
    const int n_chunks = (S + kChunk - 1) / kChunk;
    const size_t nrec = chunk == kChunk ? (size_t)n_chunks * Hv * kCRec : 0;
    const size_t rec_off = (2 * nqk + 3 * ng + 63) & ~(size_t)63;   // 256-byte aligned records
    float* ws = static_cast<float*>(workspace((rec_off + nrec) * sizeof(float), st));
    if (!ws) return ANELM_ENOMEM;
    float* qn = ws;
    float* kn = qn + nqk;
    float* beta = kn + nqk;
    float* decay = beta + ng;
    float* ldecay = decay + ng;
    float* rec = ws + rec_off;
    hipLaunchKernelGGL(dn_prep_kernel, dim3(S, Hk), dim3(kDK), 0, st, qn, kn, beta, decay, ldecay, q, k, a,
                       b, A, dt_bias, Hk, Hv, flags);
    ANELM_LAUNCHED("dn_prep_kernel");
    if (chunk == 1) {
        hipLaunchKernelGGL(dn_scan_kernel, dim3(kDV / kScanCB, Hv), dim3(kScanNT), 0, st, y, state, qn,
                           kn, v, beta, decay, S, Hk, Hv, flags);
        ANELM_LAUNCHED("dn_scan_kernel");
        return ANELM_OK;
    }
    if (flags & ANELM_DN_ORDER_TRANSFORMERS)
        hipLaunchKernelGGL(dn_chunk_pre_kernel<true>, dim3(n_chunks, Hv), dim3(kPreNT), 0, st, rec, qn, kn,
                           v, beta, ldecay, S, Hk, Hv);
    else
        hipLaunchKernelGGL(dn_chunk_pre_kernel<false>, dim3(n_chunks, Hv), dim3(kPreNT), 0, st, rec, qn, kn,
                           v, beta, ldecay, S, Hk, Hv);
    ANELM_LAUNCHED("dn_chunk_pre_kernel");
    // grid = Hv * kSlabs, a multiple of 8 (XCD mapping inside the kernel)
    hipLaunchKernelGGL(dn_chunk_seq_kernel, dim3(kSlabs * Hv), dim3(kSeqNT), 0, st, y, state, rec, S, Hv,
                       n_chunks);
    ANELM_LAUNCHED("dn_chunk_seq_kernel");
    return ANELM_OK;
}
