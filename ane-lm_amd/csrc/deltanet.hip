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
    int w_heads;   // A / dt_bias hold w_heads entries: head h uses entry h % w_heads
    // conv prologue (qwen3_5.cpp:867-874): q, k, v are channels of the raw
    // mixed projection `mix`, passed through the conv ring and SiLU here
    const float* mix;       // [2*Hk*dk + Hv*dv]
    float* conv_state;      // [2*Hk*dk + Hv*dv][conv_k - 1]
    const float* conv_w;    // [2*Hk*dk + Hv*dv][conv_k]
    int conv_pos, conv_k;
    uint32_t* readers_done; // [Hk] zeroed counters: workgroups done reading a key head's ring
    int readers;            // workgroups that read one key head's q/k channels
};

// conv1d_update for one channel (core/cpu_ops.cpp:89-129): the K-1 ring
// entries oldest first from `pos`, then the new input; followed by SiLU
// (silu_vec_inplace, cpu_ops.cpp:6-13: x / (1 + exp(-x))).  The ring write
// of the new input is left to the caller (it may be shared by workgroups).
__device__ __forceinline__ float conv_silu(const DnParams& p, int c, float xc) {
    const int sl = p.conv_k - 1;
    const float* st = p.conv_state + (size_t)c * sl;
    const float* w = p.conv_w + (size_t)c * p.conv_k;
    float sum = 0.f;
    int idx = p.conv_pos;
    for (int j = 0; j < sl; j++) {
        sum += st[idx] * w[j];
        idx = idx + 1 == sl ? 0 : idx + 1;
    }
    const float y = sum + xc * w[sl];
    return y / (expf(-y) + 1.0f);
}

// CB state columns per workgroup of NT threads: thread t owns column
// t % CB for rows [(t / CB) * RPT, +RPT).
// CONV: the inputs come from the raw projection through conv_silu; each
// value channel is read by exactly one workgroup, which also writes its ring
// slot; a key head's q/k channels are read by `readers` workgroups, and the
// last of them to finish reading (counter) writes their ring slots.
template <int CB, int NT, bool GATED, bool CONV = false>
__global__ __launch_bounds__(NT) void deltanet_decode_kernel(const DnParams p) {
    constexpr int RC = NT / CB;       // row chunks
    constexpr int RPT = kDK / RC;     // rows per thread
    static_assert(!GATED || CB == kDV, "the gated epilogue needs the whole head");
    __shared__ float qs[kDK], ks[kDK];
    __shared__ float red_a[RC][CB];
    __shared__ float red[NT / 64];
    __shared__ float vs[CB];
    __shared__ int last_reader;

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
    float qv = 0.f, kv = 0.f, qx = 0.f, kx = 0.f;
    if constexpr (CONV) {
        // channels: Q [Hk][dk] | K [Hk][dk] | V [Hv][dv] (qwen3_5.cpp:872-874)
        const int cq = kh * kDK + tid, ck = p.Hk * kDK + kh * kDK + tid;
        if (tid < kDK) {
            qx = p.mix[cq];
            kx = p.mix[ck];
            qv = conv_silu(p, cq, qx);
            kv = conv_silu(p, ck, kx);
        }
        if (tid < CB) {
            const int cv = 2 * p.Hk * kDK + h * kDV + j;
            const float vx = p.mix[cv];
            vs[tid] = conv_silu(p, cv, vx);
            p.conv_state[(size_t)cv * (p.conv_k - 1) + p.conv_pos] = vx;   // this workgroup is its only reader
        }
        // the key head's q/k ring slots take their new inputs at the end of
        // the kernel, off the path of the recurrence
    } else if (tid < kDK) {
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
    const int hw = h % p.w_heads;
    const float sp = logf(1.0f + expf(p.a[h] + p.dt_bias[hw]));
    const float decay = expf(-p.A[hw] * sp);
    const bool tf = (p.flags & ANELM_DN_ORDER_TRANSFORMERS) != 0;
    float vj = 0.f;
    if constexpr (!CONV) vj = p.v[(size_t)h * kDV + j];
    __syncthreads();
    if constexpr (CONV) vj = vs[c];

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
    if constexpr (CONV) {
        // Every ring read of this workgroup returned long ago (the values fed
        // the recurrence): count the workgroup as done with its key head; the
        // last of the head's readers stores the new q/k inputs into the ring
        // and re-zeroes the counter.  No data of this workgroup is published
        // through the counter, so it is relaxed.
        __syncthreads();
        if (tid == 0) {
            const uint32_t n = __hip_atomic_fetch_add(p.readers_done + kh, 1u, __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT);
            last_reader = n == (uint32_t)p.readers - 1u;
            if (last_reader) __hip_atomic_store(p.readers_done + kh, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        __syncthreads();
        if (last_reader && tid < kDK) {
            const int sl = p.conv_k - 1;
            p.conv_state[(size_t)(kh * kDK + tid) * sl + p.conv_pos] = qx;
            p.conv_state[(size_t)(p.Hk * kDK + kh * kDK + tid) * sl + p.conv_pos] = kx;
        }
    }
}

// ---------------------------------------------------------------- prefill
// Pre-pass: per (token, key head) l2-normalise q and k and scale q
// (qwen3_5.cpp:879-887); per (token, value head) beta and decay
// (qwen3_5.cpp:896-898).
// One wave per (token, key head) row, four rows per workgroup; each lane
// holds two adjacent elements and the norms reduce within the wave.
constexpr int kPrepRows = 4;
__global__ __launch_bounds__(64 * kPrepRows) void dn_prep_kernel(float* qn, float* kn, float* beta, float* decay,
                                                                 float* ldecay, const float* q, const float* k,
                                                                 const float* a, const float* b, const float* A,
                                                                 const float* dt_bias, int S, int Hk, int Hv,
                                                                 int flags) {
    const int row = blockIdx.x * kPrepRows + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (row >= S * Hk) return;   // (no barrier in this kernel)
    const int t = row / Hk, kh = row % Hk;
    const size_t off = (size_t)row * kDK + 2 * lane;
    float2 qv = *reinterpret_cast<const float2*>(q + off), kv = *reinterpret_cast<const float2*>(k + off);
    if (flags & ANELM_DN_L2NORM) {
        float sq = qv.x * qv.x + qv.y * qv.y, sk = kv.x * kv.x + kv.y * kv.y;
#pragma unroll
        for (int m = 1; m < 64; m <<= 1) {
            sq += __shfl_xor(sq, m, 64);
            sk += __shfl_xor(sk, m, 64);
        }
        const float iq = 1.0f / sqrtf(sq + 1e-12f), ik = 1.0f / sqrtf(sk + 1e-12f);
        qv = make_float2(qv.x * iq, qv.y * iq);
        kv = make_float2(kv.x * ik, kv.y * ik);
    }
    const float qs = 1.0f / sqrtf((float)kDK);
    *reinterpret_cast<float2*>(qn + off) = make_float2(qv.x * qs, qv.y * qs);
    *reinterpret_cast<float2*>(kn + off) = kv;
    const int group = Hv / Hk;
    for (int gi = lane; gi < group; gi += 64) {
        const int h = kh * group + gi;
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
// is computed for all chunks at once (dn_chunk_prep_mfma_kernel), and
// dn_chunk_mfma_kernel then carries the state through the chunks.  Decay
// ratios are formed in log space (all exponents <= 0).  Rows past the
// sequence end are zero (beta 0, log decay 0), so they change nothing.
constexpr int kChunk = 64;
constexpr int kCMat = kChunk * kDK;             // floats per chunk matrix
constexpr int kCRec = 5 * kCMat + 64;           // Ut, Wm, Op, Qh, Kh, gC

// ------------------------------------------- chunk preparation on fp32 MFMA
// The per-chunk matrices above, on v_mfma_f32_16x16x4_f32, from the raw
// inputs: the pre-pass of the token scan (dn_prep_kernel: l2 norm and q scale,
// beta, log decay) is folded in, so q and k are read once and nothing is
// staged through memory.
// One workgroup (8 waves) per (chunk, key head); the key head's G = Hv / Hk
// value heads share its key and query rows, so the Gram tiles K K^T and Q K^T
// (the 10 lower 16x16 tiles of each) are computed once and kept in registers.
// Per value head:
//   Am = -A (strictly lower, row-major) and P (lower) go to LDS;
//   wave 0 turns the diagonal 16x16 blocks of Am into T_rr = (I + A_rr)^-1
//   by substitution, in place;
//   for B = [beta V | beta exp(lgT) K] (64 x 256) the blocked forward
//   substitution and the product with P run per 16-column tile of B (wave w
//   owns tiles 2w, 2w + 1; it loads its tiles of B straight into the
//   accumulator layout: V columns from memory, K columns from LDS):
//     X_r = T_rr (B_r + sum_{s<r} Am_rs X_s),  Y_r = sum_{s<=r} P_rs X_s
//   with X = [Ut | Wm] and Y = [Op | P Wm] (Qh = diag(exp(lg)) Q - P Wm).
// MFMA operand layouts as in dn_chunk_mfma_kernel: A[m][k] in lane m + 16 k,
// B[k][n] in lane n + 16 k, D[m][n] in lane n + 16 (m / 4), element m % 4.
// The contraction index of k-step e is 4 k + e in both operands, so an A
// operand is one 16-byte LDS read per lane for four MFMAs, and a result tile
// in the D layout is already the B operand of the next product: X stays in
// registers from its substitution to its product with P.
// LDS matrices are row-major with 16-byte chunks XOR-swizzled by (row & 15);
// 66 KB, so two workgroups share a CU (one's serial phases overlap the other).
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
constexpr int kPmNT = 512;
constexpr int kPmK = 0;                        // K rows [64][128]
constexpr int kPmR = kCMat;                    // Q rows [64][128] for the Gram tiles, then:
constexpr int kPmA = kPmR;                     //   Am [64][64] (T_rr on its diagonal blocks)
constexpr int kPmP = kPmA + kChunk * kChunk;   //   P [64][64]
constexpr int kPmLg = kPmR + kCMat;            // lg[65] (+3 pad)
constexpr int kPmBt = kPmLg + 68;              // beta[64]
constexpr int kPmQs = kPmBt + kChunk;          // q row scale[64] (l2 norm and 1/sqrt(dk))
constexpr int kPmEb = kPmQs + kChunk;          // exp(lg[t + 1]) (decay-first) or exp(lg[t]): scales K in B
constexpr int kPmEq = kPmEb + kChunk;          // exp(lg[t + 1]): scales q in Qh
constexpr int kPmEk = kPmEq + kChunk;          // exp(lg_L - lg[t + 1]): scales K in Kh
constexpr int kPmLds = (kPmEk + kChunk) * 4;

__device__ __forceinline__ int sw128(int t, int d) { return t * kDK + 4 * ((d >> 2) ^ (t & 15)) + (d & 3); }
__device__ __forceinline__ int sw64(int r, int c) { return r * kChunk + 4 * ((c >> 2) ^ (r & 15)) + (c & 3); }

template <bool TF>
__global__ __launch_bounds__(kPmNT, 2) void dn_chunk_prep_mfma_kernel(
    float* __restrict__ rec, const float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
    const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ A,
    const float* __restrict__ dt_bias, int S, int Hk, int Hv, int flags) {
    extern __shared__ __attribute__((aligned(16))) float sm[];
    float* Ks = sm + kPmK;
    float* Rs = sm + kPmR;
    float* Am = sm + kPmA;
    float* Pm = sm + kPmP;
    float* lg = sm + kPmLg;
    float* bt = sm + kPmBt;
    float* qs = sm + kPmQs;
    float* eb = sm + kPmEb;
    float* eq = sm + kPmEq;
    float* ek = sm + kPmEk;
    const int c = blockIdx.x, kh = blockIdx.y, tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lm = lane & 15, lk = lane >> 4;
    const int G = Hv / Hk;
    const int t0 = c * kChunk, L = min(kChunk, S - t0);
    // ---- key and query rows of the chunk, l2-normalised (qwen3_5.cpp:879-887),
    // q also scaled by 1/sqrt(dk); zero past the sequence end.  A row is 32
    // float4 chunks held by 32 consecutive lanes (half a wave)
    {
        float4 kv[4], qv[4];
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const int e = tid + kPmNT * x, t = e >> 5, ch = e & 31;
            const size_t off = ((size_t)(t0 + min(t, L - 1)) * Hk + kh) * kDK + 4 * ch;
            kv[x] = *reinterpret_cast<const float4*>(k + off);
            qv[x] = *reinterpret_cast<const float4*>(q + off);
        }
        const float qk_scale = 1.0f / sqrtf((float)kDK);
#pragma unroll
        for (int x = 0; x < 4; x++) {
            const int e = tid + kPmNT * x, t = e >> 5, ch = e & 31;
            float ik = 1.f, iq = 1.f;
            if (flags & ANELM_DN_L2NORM) {
                float sk = kv[x].x * kv[x].x + kv[x].y * kv[x].y + kv[x].z * kv[x].z + kv[x].w * kv[x].w;
                float sq = qv[x].x * qv[x].x + qv[x].y * qv[x].y + qv[x].z * qv[x].z + qv[x].w * qv[x].w;
#pragma unroll
                for (int m = 1; m < 32; m <<= 1) {
                    sk += __shfl_xor(sk, m, 64);
                    sq += __shfl_xor(sq, m, 64);
                }
                ik = 1.0f / sqrtf(sk + 1e-12f);
                iq = 1.0f / sqrtf(sq + 1e-12f);
            }
            const float mk = t < L ? ik : 0.f, mq = t < L ? iq * qk_scale : 0.f;
            *reinterpret_cast<float4*>(Ks + sw128(t, 4 * ch)) =
                make_float4(kv[x].x * mk, kv[x].y * mk, kv[x].z * mk, kv[x].w * mk);
            *reinterpret_cast<float4*>(Rs + sw128(t, 4 * ch)) =
                make_float4(qv[x].x * mq, qv[x].y * mq, qv[x].z * mq, qv[x].w * mq);
            if (ch == 0) qs[t] = mq;
        }
    }
    lds_barrier();
    // ---- Gram tiles: 10 lower tiles of K K^T (ids 0..9) and of Q K^T (10..19);
    // wave w takes ids w, w + 8, w + 16
    v4f gram[3];
#pragma unroll
    for (int u = 0; u < 3; u++) {
        const int id = w + 8 * u;
        gram[u] = v4f{0.f, 0.f, 0.f, 0.f};
        if (id >= 20) continue;
        const int pi = id % 10, ti = (pi >= 1) + (pi >= 3) + (pi >= 6), tj = pi - ti * (ti + 1) / 2;
        const float* src = id < 10 ? Ks : Rs;
        v4f a0 = gram[u], a1 = gram[u];
#pragma unroll
        for (int x = 0; x < 8; x++) {
            const float4 a4 = *reinterpret_cast<const float4*>(src + sw128(16 * ti + lm, 16 * x + 4 * lk));
            const float4 b4 = *reinterpret_cast<const float4*>(Ks + sw128(16 * tj + lm, 16 * x + 4 * lk));
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, b4.x, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, b4.y, a1, 0, 0, 0);
            a0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, b4.z, a0, 0, 0, 0);
            a1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, b4.w, a1, 0, 0, 0);
        }
        gram[u] = a0 + a1;
        __builtin_amdgcn_sched_barrier(0);   // one tile's operands live at a time
    }
    lds_barrier();   // the query rows are no longer read: their space takes Am and P
    // rows past the sequence end fall outside these ranges and load as zeros
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(v), 0,
                                                                         (int)((size_t)S * Hv * kDV * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(q), 0,
                                                                         (int)((size_t)S * Hk * kDK * 4), 0x00020000);
    for (int g = 0; g < G; g++) {
        const int h = kh * G + g;
        float* out = rec + ((size_t)c * Hv + h) * kCRec;
        const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(out, 0, kCRec * 4, 0x00020000);
        // lane-derived addresses are recomputed per value head, not held across the loop
        int ltid = tid;
        asm volatile("" : "+v"(ltid));
        const int lane = ltid & 63, lm = lane & 15, lk = lane >> 4;
        // this wave's memory operands, issued first: V rows of its B tiles
        // (waves 0..3, tiles 0..7) or the raw q rows of its Qh tiles (waves 4..7)
        const bool wpart = w >= 4;
        float pre[2][4][4];
#pragma unroll
        for (int u = 0; u < 2; u++)
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 16 * r + 4 * lk + e, col = 16 * ((2 * w + u) & 7) + lm;
                    const int off = wpart ? ((t0 + t) * Hk + kh) * kDK + col : ((t0 + t) * Hv + h) * kDV + col;
                    pre[u][r][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(wpart ? rq : rv,
                                                                                                 off * 4, 0, 0));
                }
        // ---- beta = sigmoid(b) and log decay = -A softplus(a + dt_bias)
        // (qwen3_5.cpp:896-898); lg[t + 1] = sum_{j <= t} log decay_j (wave 0)
        if (w == 0) {
            const bool in = lane < L;
            float x = 0.f, bv = 0.f;
            if (in) {
                const size_t gi = (size_t)(t0 + lane) * Hv + h;
                bv = 1.0f / (1.0f + expf(-b[gi]));
                x = -A[h] * logf(1.0f + expf(a[gi] + dt_bias[h]));
            }
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const float y = __shfl_up(x, d, 64);
                if (lane >= d) x += y;
            }
            lg[lane + 1] = x;
            if (lane == 0) lg[0] = 0.f;
            bt[lane] = bv;
            // the per-row decay factors every lane of the value head uses
            // (the same expressions as per element, evaluated once per row)
            const float xs = __shfl_up(x, 1, 64);   // (every lane takes part in the shuffles)
            const float xl = __shfl(x, 63, 64);     // lg_L
            const float xp = lane == 0 ? 0.f : xs;  // lg[t]
            const float e1 = expf(x);
            eq[lane] = e1;
            eb[lane] = TF ? e1 : expf(xp);
            ek[lane] = expf(xl - x);
        }
        lds_barrier();
        // ---- Am = -A and P from the Gram tiles
#pragma unroll
        for (int u = 0; u < 3; u++) {
            const int id = w + 8 * u;
            if (id >= 20) continue;
            const int pi = id % 10, ti = (pi >= 1) + (pi >= 3) + (pi >= 6), tj = pi - ti * (ti + 1) / 2;
            const int i = 16 * tj + lm;
            const float lgi = lg[i + 1];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int t = 16 * ti + 4 * lk + e;
                if (id < 10) {
                    const float lgT = TF ? lg[t + 1] : lg[t];
                    Am[sw64(t, i)] = i < t ? -(bt[t] * expf(lgT - lgi) * gram[u][e]) : 0.f;
                } else {
                    Pm[sw64(t, i)] = i <= t ? expf(lg[t + 1] - lgi) * gram[u][e] : 0.f;
                }
            }
        }
        lds_barrier();
        if (w == 0) {
            // ---- T_rr = (I + A_rr)^-1 for the 4 diagonal blocks: lane 16 b + j
            // computes column j of block b by substitution, then writes it over A_rr
            const int b = lk, j = lm;
            float x[16];
#pragma unroll
            for (int t = 0; t < 16; t++) {
                float acc = t == j ? 1.f : 0.f;
#pragma unroll
                for (int i4 = 0; i4 < t; i4 += 4) {
                    const float4 a4 = *reinterpret_cast<const float4*>(Am + sw64(16 * b + t, 16 * b + i4));
                    acc = fmaf(a4.x, x[i4], acc);
                    if (i4 + 1 < t) acc = fmaf(a4.y, x[i4 + 1], acc);
                    if (i4 + 2 < t) acc = fmaf(a4.z, x[i4 + 2], acc);
                    if (i4 + 3 < t) acc = fmaf(a4.w, x[i4 + 3], acc);
                }
                x[t] = acc;
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int t = 0; t < 16; t++) Am[sw64(16 * b + t, 16 * b + j)] = x[t];
        } else {
            // ---- Kh = diag(exp(lg_L - lg)) K, stored transposed (Kh^T [128][64]:
            // the scan reads it as rows of its state-row tiles), gC (waves 1..7)
            const float lgL = lg[kChunk];
            for (int e = ltid - 64; e < kCMat / 4; e += kPmNT - 64) {
                const int kd = e >> 4, t4 = e & 15;
                v4f o4;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    const int t = 4 * t4 + j;
                    o4[j] = Ks[sw128(t, kd)] * ek[t];
                }
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, o4), ro,
                                                       (4 * kCMat + kd * kChunk + 4 * t4) * 4, 0, 0);
            }
            if (ltid == 64)
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, expf(lgL)), ro, 5 * kCMat * 4, 0, 0);
        }
        lds_barrier();
        // ---- X and Y for column tiles jt = 2w + u of B
        v4f X[2][4];
#pragma unroll
        for (int r = 0; r < 4; r++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const int jt = 2 * w + u;
                // B_r of this tile in the accumulator layout: rows 16 r + 4 lk + e, column lm
                v4f acc;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 16 * r + 4 * lk + e;
                    acc[e] = bt[t] * (wpart ? Ks[sw128(t, 16 * (jt - 8) + lm)] * eb[t] : pre[u][r][e]);
                }
#pragma unroll
                for (int s2 = 0; s2 < r; s2++) {
                    const float4 a4 = *reinterpret_cast<const float4*>(Am + sw64(16 * r + lm, 16 * s2 + 4 * lk));
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.x, X[u][s2][0], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.y, X[u][s2][1], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.z, X[u][s2][2], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a4.w, X[u][s2][3], acc, 0, 0, 0);
                }
                const float4 t4 = *reinterpret_cast<const float4*>(Am + sw64(16 * r + lm, 16 * r + 4 * lk));
                v4f xr = {0.f, 0.f, 0.f, 0.f};
                xr = __builtin_amdgcn_mfma_f32_16x16x4f32(t4.x, acc[0], xr, 0, 0, 0);
                xr = __builtin_amdgcn_mfma_f32_16x16x4f32(t4.y, acc[1], xr, 0, 0, 0);
                xr = __builtin_amdgcn_mfma_f32_16x16x4f32(t4.z, acc[2], xr, 0, 0, 0);
                xr = __builtin_amdgcn_mfma_f32_16x16x4f32(t4.w, acc[3], xr, 0, 0, 0);
                X[u][r] = xr;
                // Y_r = sum_{s <= r} P_rs X_s
                v4f y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s2 = 0; s2 <= r; s2++) {
                    const float4 p4 = *reinterpret_cast<const float4*>(Pm + sw64(16 * r + lm, 16 * s2 + 4 * lk));
                    y = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.x, X[u][s2][0], y, 0, 0, 0);
                    y = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.y, X[u][s2][1], y, 0, 0, 0);
                    y = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.z, X[u][s2][2], y, 0, 0, 0);
                    y = __builtin_amdgcn_mfma_f32_16x16x4f32(p4.w, X[u][s2][3], y, 0, 0, 0);
                }
                // rows t = 16 r + 4 lk + e, column 16 (jt % 8) + lm of Ut / Wm and Op / Qh
                const int col = 16 * (jt & 7) + lm;
                const int ox = wpart ? kCMat : 0, oy = wpart ? 3 * kCMat : 2 * kCMat;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const int t = 16 * r + 4 * lk + e;
                    // through a scalar: a bit_cast of a vector element is lowered as element 0
                    const float xv = xr[e];
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, xv), ro, (ox + t * kDK + col) * 4,
                                                          0, 0);
                    float yv = y[e];
                    if (wpart) yv = eq[t] * (qs[t] * pre[u][r][e]) - yv;
                    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, yv), ro, (oy + t * kDK + col) * 4,
                                                          0, 0);
                }
                __builtin_amdgcn_sched_barrier(0);   // bounds the loads hoisted ahead of this tile
            }
        }
        lds_barrier();   // Am, P, lg and beta are rewritten for the next value head
    }
}

// The state is carried through the chunks in slabs of 16 columns (8 per head).
constexpr int kSeqCB = 16;
constexpr int kSlabs = kDV / kSeqCB;

// ------------------------------------------------ chunk scan on fp32 MFMA
// The same three products per chunk on v_mfma_f32_16x16x4_f32 (fp32 inputs,
// fp32 accumulation).  A workgroup (8 waves, two per SIMD) owns a 16-column
// slab of one head's state, kept in LDS column-major (Sc[c][i]):
//   waves 0-3: X = Wm S0 for chunk rows [16 w, 16 w + 16), U = Ut - X (LDS);
//   waves 4-7: Y = Qh S0 for chunk rows [16 (w - 4), ...), y = Op + Y (LDS,
//   then stored by all 8 waves);
//   then wave w: S = gC S0 + Kh^T U for state rows [16 w, 16 w + 16).
// Every operand but the state and U is read by one wave only (its Wm or Qh
// rows, its Kh^T rows, its Ut or Op entries), so it goes from memory straight
// into registers, the next chunk's loads spread over this chunk's products;
// LDS carries only the state slab and U.
// MFMA operand layouts (16x16x4, one block): A[m][k] in lane m + 16 k,
// B[k][n] in lane n + 16 k, D[m][n] in lane n + 16 (m / 4), element m % 4.
// The contraction index is permuted identically in both operands: lane (m, k)
// of k-step (x, e) takes state row (or chunk row) 16 x + 4 k + e, so an A
// operand is one 16-byte read per lane for four k-steps.
constexpr int kMsNT = 512;
constexpr int kScP = kDK + 4;        // Sc row pitch (floats): 16-byte reads of 16 lanes hit distinct banks
constexpr int kUlP = kSeqCB + 4;     // U row pitch: rows 4 apart land 16 banks apart
constexpr int kMsLds = (kSeqCB * kScP + 2 * kChunk * kUlP) * 4;

// One wave's operands of one chunk.
struct ScanOps {
    v4f m[8];     // Wm (waves 0-3) or Qh (4-7) row 16 (w & 3) + lr, state rows 16 x + 4 lq + (0..3)
    v4f kt[4];    // Kh^T row 16 w + lr, chunk rows 16 x + 4 lq + (0..3)
    float uo[4];  // Ut (waves 0-3) or Op (4-7) at chunk row 16 (w & 3) + 4 lq + j, slab column lr
    float gc;
};

// Where one wave's operands of chunk ch lie: one chunk record per buffer
// resource (offsets stay small for any sequence length).
struct ScanSrc {
    __amdgpu_buffer_rsrc_t rr;
    int mo, ko, uo;   // float offsets of this lane's first Wm / Qh, Kh^T and Ut / Op element
};

__device__ __forceinline__ ScanSrc scan_src(const float* rec, int ch, int Hv, int h, int w, int lr, int lq, int c0) {
    ScanSrc s;
    s.rr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(rec) + ((size_t)ch * Hv + h) * kCRec, 0, kCRec * 4,
                                             0x00020000);
    const int mt = w & 3;
    s.mo = (w < 4 ? kCMat : 3 * kCMat) + (16 * mt + lr) * kDK + 4 * lq;
    s.ko = 4 * kCMat + (16 * w + lr) * kChunk + 4 * lq;
    s.uo = (w < 4 ? 0 : 2 * kCMat) + (16 * mt + 4 * lq) * kDK + c0 + lr;
    return s;
}

// Part x (0..7) of a wave's loads of one chunk: m[x], then kt[x] (x < 4) or
// uo[x - 4] (x >= 4), and gc with the last part.  The parts are issued
// between the MFMA groups of the previous chunk's products: issued all at
// once, the workgroup's loads fill the CU's memory queue and the waves stall
// at their next memory instruction instead of computing.
__device__ __forceinline__ void scan_part(ScanOps& o, const ScanSrc& s, int x) {
    o.m[x] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(s.rr, (s.mo + 16 * x) * 4, 0, 0));
    if (x < 4)
        o.kt[x] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(s.rr, (s.ko + 16 * x) * 4, 0, 0));
    else
        o.uo[x - 4] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s.rr, (s.uo + (x - 4) * kDK) * 4, 0, 0));
    if (x == 7) o.gc = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(s.rr, 5 * kCMat * 4, 0, 0));
}

__global__ __launch_bounds__(kMsNT) __attribute__((amdgpu_waves_per_eu(2, 2))) void dn_chunk_mfma_kernel(
    float* __restrict__ y, float* __restrict__ state, const float* __restrict__ rec, int S, int Hv, int n_chunks) {
    extern __shared__ __attribute__((aligned(16))) float smem[];
    float (*Sc)[kScP] = reinterpret_cast<float (*)[kScP]>(smem);                   // state slab
    float (*Ul)[kUlP] = reinterpret_cast<float (*)[kUlP]>(smem + kSeqCB * kScP);   // U of the chunk
    float (*Yl)[kUlP] = Ul + kChunk;                                               // its y tile
    // XCD-aware: the 8 slabs of a head share its chunk records, so they go to
    // one XCD (workgroup id mod 8 selects the XCD; Hv * 8 workgroups)
    const int nwg = gridDim.x, id = blockIdx.x;
    const int per_xcd = nwg / 8, k8 = id / 8, xcd = id % 8;
    const int h = (xcd * per_xcd + k8) / kSlabs, slab = (xcd * per_xcd + k8) % kSlabs;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15, lq = lane >> 4;
    const int mt = w & 3;
    const int c0 = slab * kSeqCB;
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(y, 0, (int)((size_t)S * Hv * kDV * 4), 0x00020000);

    // two operand sets, A and B: a chunk is computed from one while the next
    // chunk's loads land in the other (no register copies between them)
    ScanOps opA, opB;
    {
        const ScanSrc s0 = scan_src(rec, 0, Hv, h, w, lr, lq, c0);
#pragma unroll
        for (int x = 0; x < 8; x++) scan_part(opA, s0, x);
    }
    float* Sp = state + (size_t)h * kDK * kDV;
    for (int e = tid; e < kDK * kSeqCB; e += kMsNT) {
        const int i = e / kSeqCB, c = e % kSeqCB;
        Sc[c][i] = Sp[(size_t)i * kDV + c0 + c];
    }
    __syncthreads();

    auto chunk = [&](const ScanOps& cur, ScanOps& nxt, int ch) __attribute__((always_inline)) {
        // the next chunk's operands (the last chunk reloads its own: no branch)
        const ScanSrc src = scan_src(rec, ch + 1 < n_chunks ? ch + 1 : ch, Hv, h, w, lr, lq, c0);
        // ---- X = Wm S0 (waves 0-3) or Y = Qh S0 (waves 4-7): 32 MFMAs in 4
        // chains, one part of the next chunk's loads ahead of each group of 4
        v4f sb[8];
#pragma unroll
        for (int x = 0; x < 8; x++) sb[x] = *reinterpret_cast<const v4f*>(&Sc[lr][16 * x + 4 * lq]);
        v4f Z[4];
#pragma unroll
        for (int e = 0; e < 4; e++) Z[e] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int x = 0; x < 8; x++) {
            scan_part(nxt, src, x);
            __builtin_amdgcn_sched_barrier(0);   // the part is issued here, not hoisted or sunk
#pragma unroll
            for (int e = 0; e < 4; e++)
                Z[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.m[x][e], sb[x][e], Z[e], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        const v4f Zs = (Z[0] + Z[1]) + (Z[2] + Z[3]);
        // element j is chunk row 16 mt + 4 lq + j, slab column lr:
        // U = Ut - X (waves 0-3) and y = Op + Y (waves 4-7) go to LDS
        {
            float (*dst)[kUlP] = w < 4 ? Ul : Yl;
            const float sg = w < 4 ? -1.f : 1.f;
#pragma unroll
            for (int j = 0; j < 4; j++) dst[16 * mt + 4 * lq + j][lr] = cur.uo[j] + sg * Zs[j];
        }
        lds_barrier();   // U and y complete; every wave's reads of S0 are done
        {
            // the y tile to memory, one 8-byte store per lane of every wave:
            // all waves then have the same memory operations in flight, so the
            // waits for this chunk's operands count the same everywhere
            // (y rows past S fall out of the buffer range and are dropped)
            const int t = tid >> 3, cp = tid & 7;
            const float2 yv = *reinterpret_cast<const float2*>(&Yl[t][2 * cp]);
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, yv), ry,
                                                  (((ch * kChunk + t) * Hv + h) * kDV + c0 + 2 * cp) * 4, 0, 0);
        }
        // ---- S = gC S0 + Kh^T U for state rows 16 w + (0..15): 16 MFMAs in 4 chains
        float ub[16];
#pragma unroll
        for (int s = 0; s < 16; s++) ub[s] = Ul[16 * (s >> 2) + 4 * lq + (s & 3)][lr];
        v4f* srow = reinterpret_cast<v4f*>(&Sc[lr][16 * w + 4 * lq]);
        v4f Sn[4];
        Sn[0] = cur.gc * *srow;
#pragma unroll
        for (int e = 1; e < 4; e++) Sn[e] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int x = 0; x < 4; x++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                Sn[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(cur.kt[x][e], ub[4 * x + e], Sn[e], 0, 0, 0);
        // rows written here are read (as C) only by this wave
        *srow = (Sn[0] + Sn[1]) + (Sn[2] + Sn[3]);
        lds_barrier();   // new state complete, U and y consumed
    };
    // pairs of chunks, then an odd last one: inside the loop both halves run
    // unconditionally, so the loads a half issues for the other are not sunk
    // into a conditional block next to their use
    int ch = 0;
    for (; ch + 1 < n_chunks; ch += 2) {
        chunk(opA, opB, ch);
        chunk(opB, opA, ch + 1);
    }
    if (ch < n_chunks) chunk(opA, opB, ch);
    for (int e = tid; e < kDK * kSeqCB; e += kMsNT) {
        const int i = e / kSeqCB, c = e % kSeqCB;
        Sp[(size_t)i * kDV + c0 + c] = Sc[c][i];
    }
}

}  // namespace
}  // namespace anelm

using namespace anelm;

namespace anelm {
namespace {
int deltanet_decode_impl(float* y, float* state, const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A, const float* dt_bias, const float* z, const float* norm_w,
                         int n_seqs, int Hk, int Hv, int dk, int dv, int flags, hipStream_t st);
}  // namespace
}  // namespace anelm

extern "C" int anelm_deltanet_decode(float* y, float* state, const float* q, const float* k,
                                     const float* v, const float* a, const float* b,
                                     const float* A, const float* dt_bias, const float* z,
                                     const float* norm_w, int Hk, int Hv, int dk, int dv,
                                     int flags, void* stream) {
    return deltanet_decode_impl(y, state, q, k, v, a, b, A, dt_bias, z, norm_w, 1, Hk, Hv, dk, dv, flags,
                                as_stream(stream));
}

extern "C" int anelm_deltanet_decode_batched(float* y, float* state, const float* q, const float* k,
                                             const float* v, const float* a, const float* b,
                                             const float* A, const float* dt_bias, const float* z,
                                             const float* norm_w, int n_seqs, int Hk, int Hv, int dk,
                                             int dv, int flags, void* stream) {
    return deltanet_decode_impl(y, state, q, k, v, a, b, A, dt_bias, z, norm_w, n_seqs, Hk, Hv, dk, dv, flags,
                                as_stream(stream));
}

namespace anelm {
namespace {
// n_seqs sequences of Hk key / Hv value heads as one launch over n_seqs * Hv
// heads: sequence s's value head j is head s*Hv + j, its key head
// s*Hk + j/(Hv/Hk) -- the same h / (Hv/Hk) mapping over the stacked heads --
// and A / dt_bias (layer weights) are shared by the sequences.
int deltanet_decode_impl(float* y, float* state, const float* q, const float* k, const float* v, const float* a,
                         const float* b, const float* A, const float* dt_bias, const float* z, const float* norm_w,
                         int n_seqs, int Hk, int Hv, int dk, int dv, int flags, hipStream_t st) {
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
    ANELM_REQUIRE(n_seqs > 0 && (long)n_seqs * Hv <= 65535, "deltanet_decode: %d sequences x %d value heads "
                  "(at most 65535 heads per launch)", n_seqs, Hv);
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
    p.Hk = Hk * n_seqs;
    p.Hv = Hv * n_seqs;
    p.w_heads = Hv;
    p.flags = flags;
    if (flags & ANELM_DN_GATED_NORM) {
        ANELM_NONNULL(z);
        ANELM_NONNULL(norm_w);
        p.z = z;
        p.norm_w = norm_w;
        hipLaunchKernelGGL((deltanet_decode_kernel<128, 512, true>), dim3(1, p.Hv), dim3(512), 0, st, p);
    } else {
        hipLaunchKernelGGL((deltanet_decode_kernel<32, 256, false>), dim3(kDV / 32, p.Hv), dim3(256), 0,
                           st, p);
    }
    ANELM_LAUNCHED("deltanet_decode_kernel");
    return ANELM_OK;
}
}  // namespace
}  // namespace anelm

extern "C" int anelm_deltanet_decode_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                                               const float* proj, const float* conv_w, const float* A,
                                               const float* dt_bias, const float* norm_w, int Hk, int Hv,
                                               int dk, int dv, int conv_kernel, int flags, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_NONNULL(conv_state);
    ANELM_NONNULL(conv_pos);
    ANELM_NONNULL(proj);
    ANELM_NONNULL(conv_w);
    ANELM_NONNULL(A);
    ANELM_NONNULL(dt_bias);
    ANELM_REQUIRE(dk == kDK && dv == kDV, "deltanet_decode_from_proj: dk=%d dv=%d (only 128x128)", dk, dv);
    ANELM_REQUIRE(Hk > 0 && Hv > 0 && Hv % Hk == 0 && Hv <= 65535,
                  "deltanet_decode_from_proj: Hv %d not a multiple of Hk %d", Hv, Hk);
    ANELM_REQUIRE(conv_kernel >= 2 && conv_kernel <= 16, "deltanet_decode_from_proj: conv kernel %d",
                  conv_kernel);
    ANELM_REQUIRE(*conv_pos >= 0 && *conv_pos < conv_kernel - 1, "deltanet_decode_from_proj: conv_pos %d",
                  *conv_pos);
    ANELM_REQUIRE((flags & ~7) == 0, "deltanet_decode_from_proj: unknown flags 0x%x", flags);
    const bool gated = (flags & ANELM_DN_GATED_NORM) != 0;
    ANELM_REQUIRE(!gated || norm_w != nullptr, "deltanet_decode_from_proj: GATED_NORM needs norm_w");
    hipStream_t st = as_stream(stream);
    uint32_t* ctr = counters((size_t)Hk, kCtrDeltaNetConv, st);
    if (!ctr) return ANELM_ERANGE;
    const long qkv = 2L * Hk * kDK + (long)Hv * kDV;
    DnParams p{};
    p.y = y;
    p.state = state;
    p.z = proj + qkv;                       // [Hv][dv]
    p.a = p.z + (long)Hv * kDV;             // [Hv]
    p.b = p.a + Hv;                         // [Hv]
    p.A = A;
    p.dt_bias = dt_bias;
    p.norm_w = norm_w;
    p.Hk = Hk;
    p.Hv = Hv;
    p.w_heads = Hv;
    p.flags = flags;
    p.mix = proj;
    p.conv_state = conv_state;
    p.conv_w = conv_w;
    p.conv_pos = *conv_pos;
    p.conv_k = conv_kernel;
    p.readers_done = ctr;
    if (gated) {
        p.readers = Hv / Hk;
        hipLaunchKernelGGL((deltanet_decode_kernel<128, 512, true, true>), dim3(1, Hv), dim3(512), 0, st, p);
    } else {
        p.readers = (Hv / Hk) * (kDV / 32);
        hipLaunchKernelGGL((deltanet_decode_kernel<32, 256, false, true>), dim3(kDV / 32, Hv), dim3(256), 0, st,
                           p);
    }
    ANELM_LAUNCHED("deltanet_decode_kernel (conv prologue)");
    int np = *conv_pos + 1;
    if (np == conv_kernel - 1) np = 0;
    *conv_pos = np;
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
    ANELM_REQUIRE((size_t)(S + kChunk) * Hv * kDV * sizeof(float) < 0x7fffffffu,
                  "deltanet_prefill: %d tokens x %d heads exceed the 2 GiB output range", S, Hv);
    ANELM_REQUIRE((flags & ~3) == 0, "deltanet_prefill: flags 0x%x (GATED_NORM is decode-only)", flags);
    if (S == 0) return ANELM_OK;
    hipStream_t st = as_stream(stream);
    if (chunk == 1) {
        const size_t nqk = (size_t)S * Hk * kDK, ng = (size_t)S * Hv;
        float* ws = static_cast<float*>(workspace((2 * nqk + 3 * ng) * sizeof(float), st));
        if (!ws) return ANELM_ENOMEM;
        float* qn = ws;
        float* kn = qn + nqk;
        float* beta = kn + nqk;
        float* decay = beta + ng;
        float* ldecay = decay + ng;
        hipLaunchKernelGGL(dn_prep_kernel, dim3((S * Hk + kPrepRows - 1) / kPrepRows), dim3(64 * kPrepRows), 0, st,
                           qn, kn, beta, decay, ldecay, q, k, a, b, A, dt_bias, S, Hk, Hv, flags);
        ANELM_LAUNCHED("dn_prep_kernel");
        hipLaunchKernelGGL(dn_scan_kernel, dim3(kDV / kScanCB, Hv), dim3(kScanNT), 0, st, y, state, qn,
                           kn, v, beta, decay, S, Hk, Hv, flags);
        ANELM_LAUNCHED("dn_scan_kernel");
        return ANELM_OK;
    }
    const int n_chunks = (S + kChunk - 1) / kChunk;
    float* rec = static_cast<float*>(workspace((size_t)n_chunks * Hv * kCRec * sizeof(float), st));
    if (!rec) return ANELM_ENOMEM;
    static bool pm_attr = false;
    if (!pm_attr) {
        ANELM_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&dn_chunk_prep_mfma_kernel<true>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kPmLds));
        ANELM_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&dn_chunk_prep_mfma_kernel<false>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kPmLds));
        pm_attr = true;
    }
    if (flags & ANELM_DN_ORDER_TRANSFORMERS)
        hipLaunchKernelGGL(dn_chunk_prep_mfma_kernel<true>, dim3(n_chunks, Hk), dim3(kPmNT), kPmLds, st, rec, q, k, v,
                           a, b, A, dt_bias, S, Hk, Hv, flags);
    else
        hipLaunchKernelGGL(dn_chunk_prep_mfma_kernel<false>, dim3(n_chunks, Hk), dim3(kPmNT), kPmLds, st, rec, q, k,
                           v, a, b, A, dt_bias, S, Hk, Hv, flags);
    ANELM_LAUNCHED("dn_chunk_prep_mfma_kernel");
    // grid = Hv * kSlabs, a multiple of 8 (XCD mapping inside the kernel)
    static bool ms_attr = false;
    if (!ms_attr) {
        ANELM_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(&dn_chunk_mfma_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize, kMsLds));
        ms_attr = true;
    }
    hipLaunchKernelGGL(dn_chunk_mfma_kernel, dim3(kSlabs * Hv), dim3(kMsNT), kMsLds, st, y, state, rec, S, Hv,
                       n_chunks);
    ANELM_LAUNCHED("dn_chunk_mfma_kernel");
    return ANELM_OK;
}
