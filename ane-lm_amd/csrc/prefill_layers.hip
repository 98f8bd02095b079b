// Prompt prefill of the two layer cores from their projections, over the
// layer's persistent state (the fp16 KV ring, the DeltaNet state and conv
// ring) -- what generate.cpp:55-85 gets by running the decode core once per
// prompt token (Qwen35Model::forward_batch, models/llm/qwen3_5.cpp:1164-1217,
// batches only the projections around the per-token cores).
//
// Full attention (qwen3_5.cpp:944-1002 per token):
//   1. prep: per (token, head) row, q/k RMSNorm and RoPE at the token's
//      position; q to fp16, the new keys and values to fp16 behind the
//      cached keys (gathered oldest to newest from the ring), so keys are
//      one contiguous sequence [cached | prompt];
//   2. the causal MFMA core over that sequence, query row t being key
//      len0 + t, with the output gate in its epilogue; when the ring would
//      overflow inside the prompt, row t sees only the last `capacity` keys,
//      as the sliding ring gives the decode core;
//   3. the prompt's keys that survive in the ring are written to their slots.
// Gated DeltaNet (qwen3_5.cpp:849-908 per token):
//   1. the causal conv1d over [conv ring | prompt] + SiLU per channel
//      (cpu_ops.cpp:89-129, :6-13), split into q / k / v, with z, a, b
//      gathered alongside; the ring keeps the prompt's last inputs;
//   2. the chunked prefill (l2 norm, q scale, gates, state carried through
//      the prompt);
//   3. rmsnorm_gated with z per token and value head.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

struct PrepArgs {
    const float* q_gate;       // token t, head h at q_gate + t * qs + h * 2D
    const float* k;            // token t, kv head at k + t * ks + kvh * D
    const float* v;
    long qs, ks;
    const float* q_norm_w;     // [D] or null
    const float* k_norm_w;
    const float* rope_tab;     // [rope_rows][2 rot_pairs] or null
    int rope_rows;
    uint16_t* qh;              // [S][Hq][D] fp16
    uint16_t* kall;            // [len0 + S][Hkv][D] fp16
    uint16_t* vall;
    int S, Hq, Hkv, len0, pos0, rot_pairs, rope_mode;
    float theta, eps;
};

// One wave per (token, row), four rows of one token per workgroup (the
// token's RoPE row is loaded once for them): rows 0..Hq-1 are the token's q
// heads, the rest its kv heads (with the value row converted alongside).  The
// norm and the rotation are the decode core's (models/llm/qwen3_5.cpp:952-971):
// (x * inv) * w with inv = 1 / sqrtf(ss / D + eps), pairs rotated without
// contraction.
constexpr int kPrepRowsPerWg = 4;
template <int D>
__global__ __launch_bounds__(64 * kPrepRowsPerWg) void prefill_prep_kernel(PrepArgs a) {
    __shared__ float rows[kPrepRowsPerWg][D];
    __shared__ float cs[128], sn[128];
    const int t = blockIdx.x, wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int y = blockIdx.y * kPrepRowsPerWg + wv;
    const bool live = y < a.Hq + a.Hkv;   // (a wave past the last row still meets the barriers)
    const int pos = a.pos0 + t;
    for (int j = threadIdx.x; j < a.rot_pairs; j += 64 * kPrepRowsPerWg) {
        if (a.rope_tab != nullptr && pos < a.rope_rows) {
            cs[j] = a.rope_tab[(size_t)pos * 2 * a.rot_pairs + j];
            sn[j] = a.rope_tab[(size_t)pos * 2 * a.rot_pairs + a.rot_pairs + j];
        } else {
            // the table's formula (cpu_ops.cpp:51-55) evaluated here
            const float freq = 1.0f / powf(a.theta, (float)(2 * j) / (float)(2 * a.rot_pairs));
            const float angle = (float)pos * freq;
            cs[j] = cosf(angle);
            sn[j] = sinf(angle);
        }
    }
    const bool isq = y < a.Hq;
    const int kvh = y - a.Hq;
    float* row = rows[wv];
    constexpr int E = D / 64;
    float x[E], vv[E];
    if (live) {
        const float* src = isq ? a.q_gate + t * a.qs + (long)y * 2 * D : a.k + t * a.ks + (long)kvh * D;
        const float* w = isq ? a.q_norm_w : a.k_norm_w;
#pragma unroll
        for (int e = 0; e < E; e++) x[e] = src[lane + 64 * e];
        if (!isq) {
            const float* vs = a.v + t * a.ks + (long)kvh * D;
#pragma unroll
            for (int e = 0; e < E; e++) vv[e] = vs[lane + 64 * e];
        }
        if (w != nullptr) {
            float ss = 0.f;
#pragma unroll
            for (int e = 0; e < E; e++) ss += x[e] * x[e];
            ss = wave_sum(ss);
            const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
#pragma unroll
            for (int e = 0; e < E; e++) x[e] = (x[e] * inv) * w[lane + 64 * e];
        }
#pragma unroll
        for (int e = 0; e < E; e++) row[lane + 64 * e] = x[e];
    }
    __syncthreads();
    if (live) {
        for (int j = lane; j < a.rot_pairs; j += 64) {
            const int i0 = a.rope_mode == 0 ? 2 * j : j;
            const int i1 = a.rope_mode == 0 ? 2 * j + 1 : j + a.rot_pairs;
            const float v0 = row[i0], v1 = row[i1];
            rotate_pair(row[i0], row[i1], v0, v1, cs[j], sn[j]);
        }
    }
    __syncthreads();
    if (!live) return;
    uint16_t* dst = isq ? a.qh + ((size_t)t * a.Hq + y) * D : a.kall + ((size_t)(a.len0 + t) * a.Hkv + kvh) * D;
#pragma unroll
    for (int e = 0; e < E; e++) dst[lane + 64 * e] = f2h(row[lane + 64 * e]);
    if (!isq) {
        uint16_t* vd = a.vall + ((size_t)(a.len0 + t) * a.Hkv + kvh) * D;
#pragma unroll
        for (int e = 0; e < E; e++) vd[lane + 64 * e] = f2h(vv[e]);
    }
}

// Cached keys and values oldest to newest: key i of the ring is slot
// (start + i) mod cap.  16 bytes per thread.
__global__ __launch_bounds__(256) void ring_gather_kernel(uint16_t* kall, uint16_t* vall, const uint16_t* kc,
                                                          const uint16_t* vc, long n16, int row16, int start,
                                                          int cap) {
    const long e = blockIdx.x * 256L + threadIdx.x;
    if (e >= n16) return;
    const long i = e / row16, r = e - i * row16;
    const long slot = (start + i) % cap;
    reinterpret_cast<uint4*>(kall)[e] = reinterpret_cast<const uint4*>(kc)[slot * row16 + r];
    reinterpret_cast<uint4*>(vall)[e] = reinterpret_cast<const uint4*>(vc)[slot * row16 + r];
}

// The prompt's keys t0..S-1 (those no later prompt key overwrites) into
// their ring slots: key a of [cached | prompt] lives in slot (start + a) mod
// cap, as the ring's appends place it (qwen3_5.cpp:973-983).
__global__ __launch_bounds__(256) void ring_write_kernel(uint16_t* kc, uint16_t* vc, const uint16_t* kall,
                                                         const uint16_t* vall, long n16, int row16, int t0,
                                                         int len0, int start, int cap) {
    const long e = blockIdx.x * 256L + threadIdx.x;
    if (e >= n16) return;
    const long i = e / row16, r = e - i * row16;
    const long a = len0 + t0 + i;
    const long slot = (start + a) % cap;
    reinterpret_cast<uint4*>(kc)[slot * row16 + r] = reinterpret_cast<const uint4*>(kall)[a * row16 + r];
    reinterpret_cast<uint4*>(vc)[slot * row16 + r] = reinterpret_cast<const uint4*>(vall)[a * row16 + r];
}

// ------------------------------------------------------------ DeltaNet
struct ConvArgs {
    const float* proj;         // [S][pd]: mixed qkv (C) | z (Hv dv) | a (Hv) | b (Hv)
    const float* conv_state;   // [C][K-1] ring, oldest at slot pos
    const float* conv_w;       // [C][K]
    float* q;                  // [S][Hk dk]
    float* k;
    float* v;                  // [S][Hv dv]
    float* z;
    float* a;                  // [S][Hv]
    float* b;
    int S, C, pd, pos, nqk, nz, nab;
    int tpb;                   // tokens per thread
};

// Thread = (channel, run of tpb tokens).  Channel c < C: the causal conv over
// [ring | prompt] (sum over the K-1 older inputs oldest first, then the
// current input times the last tap, as cpu_ops.cpp:89-129 evaluates it),
// SiLU (cpu_ops.cpp:6-13), written to q, k or v.  Channels past C: z, a, b
// copied to contiguous arrays.
constexpr int kConvBatch = 16;   // tokens whose inputs one thread requests at once

template <int K>
__global__ __launch_bounds__(256) void dn_conv_prefill_kernel(ConvArgs p) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int extra = p.nz + 2 * p.nab;
    if (c >= p.C + extra) return;
    const int t0 = blockIdx.y * p.tpb, t1 = min(p.S, t0 + p.tpb);
    // the inputs of kConvBatch tokens are requested together before any of
    // them is used (the stores below may alias the rows for the compiler, so
    // it would otherwise wait for each token's load in turn)
    constexpr int NB = kConvBatch;
    if (c >= p.C) {
        const int cc = c - p.C;
        for (int tb = t0; tb < t1; tb += NB) {
            float xs[NB];
#pragma unroll
            for (int u = 0; u < NB; u++) xs[u] = tb + u < t1 ? p.proj[(size_t)(tb + u) * p.pd + c] : 0.f;
#pragma unroll
            for (int u = 0; u < NB; u++) {
                const int t = tb + u;
                if (t >= t1) break;
                if (cc < p.nz) p.z[(size_t)t * p.nz + cc] = xs[u];
                else if (cc < p.nz + p.nab) p.a[(size_t)t * p.nab + cc - p.nz] = xs[u];
                else p.b[(size_t)t * p.nab + cc - p.nz - p.nab] = xs[u];
            }
        }
        return;
    }
    constexpr int sl = K - 1;
    float hist[sl];   // inputs t-sl .. t-1, oldest first
#pragma unroll
    for (int j = 0; j < sl; j++) {
        const int tt = t0 - sl + j;
        if (tt >= 0) {
            hist[j] = p.proj[(size_t)tt * p.pd + c];
        } else {
            // ring entry of input tt < 0: the ring holds inputs -sl..-1 oldest
            // first from slot pos
            int idx = p.pos + (tt + sl);
            if (idx >= sl) idx -= sl;
            hist[j] = p.conv_state[(size_t)c * sl + idx];
        }
    }
    const float* w = p.conv_w + (size_t)c * K;
    float wl[K];
#pragma unroll
    for (int j = 0; j < K; j++) wl[j] = w[j];
    for (int tb = t0; tb < t1; tb += NB) {
        float xs[NB];
#pragma unroll
        for (int u = 0; u < NB; u++) xs[u] = tb + u < t1 ? p.proj[(size_t)(tb + u) * p.pd + c] : 0.f;
#pragma unroll
        for (int u = 0; u < NB; u++) {
            const int t = tb + u;
            if (t >= t1) break;
            const float x = xs[u];
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < sl; j++) sum += hist[j] * wl[j];
            float yv = sum + x * wl[sl];
            yv = yv / (expf(-yv) + 1.0f);
#pragma unroll
            for (int j = 0; j + 1 < sl; j++) hist[j] = hist[j + 1];
            hist[sl - 1] = x;
            if (c < p.nqk) p.q[(size_t)t * p.nqk + c] = yv;
            else if (c < 2 * p.nqk) p.k[(size_t)t * p.nqk + c - p.nqk] = yv;
            else p.v[(size_t)t * (p.C - 2 * p.nqk) + c - 2 * p.nqk] = yv;
        }
    }
}

// The ring after the prompt: input t was stored at slot (pos + t) mod (K-1),
// so the last K-1 inputs (all of them when S < K-1) overwrite their slots.
__global__ __launch_bounds__(256) void dn_conv_ring_kernel(float* conv_state, const float* proj, int S, int C,
                                                           int pd, int K, int pos) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= C) return;
    const int sl = K - 1;
    for (int t = max(0, S - sl); t < S; t++) conv_state[(size_t)c * sl + (pos + t) % sl] = proj[(size_t)t * pd + c];
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_full_attn_prefill(float* out, const float* q_gate, const float* k, const float* v,
                                       int proj_stride, uint16_t* k_cache, uint16_t* v_cache, const float* q_norm_w,
                                       const float* k_norm_w, int S, int n_heads, int n_kv_heads, int head_dim,
                                       int rot_dim, int pos0, float theta, float eps, int rope_mode, int gate,
                                       const float* rope_table, int rope_rows, int* cache_start, int* cache_len,
                                       int cache_capacity, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(q_gate);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_NONNULL(k_cache);
    ANELM_NONNULL(v_cache);
    ANELM_NONNULL(cache_start);
    ANELM_NONNULL(cache_len);
    ANELM_REQUIRE(S >= 1, "full_attn_prefill: S %d", S);
    ANELM_REQUIRE(head_dim == 128 || head_dim == 256, "full_attn_prefill: head_dim %d (128, 256)", head_dim);
    ANELM_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "full_attn_prefill: heads %d/%d", n_heads,
                  n_kv_heads);
    const int G = n_heads / n_kv_heads;
    ANELM_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "full_attn_prefill: %d q heads per kv head", G);
    ANELM_REQUIRE(rot_dim >= 0 && rot_dim % 2 == 0 && rot_dim <= head_dim && rot_dim <= 256,
                  "full_attn_prefill: rot_dim %d", rot_dim);
    ANELM_REQUIRE(rope_mode == ANELM_ROPE_INTERLEAVED || rope_mode == ANELM_ROPE_HALF_SPLIT,
                  "full_attn_prefill: rope_mode %d", rope_mode);
    ANELM_REQUIRE((q_norm_w == nullptr) == (k_norm_w == nullptr), "full_attn_prefill: give both norm weights or none");
    ANELM_REQUIRE(rope_table == nullptr || rope_rows >= 0, "full_attn_prefill: rope_rows %d", rope_rows);
    ANELM_REQUIRE(proj_stride == 0 || proj_stride >= n_heads * 2 * head_dim,
                  "full_attn_prefill: proj_stride %d", proj_stride);
    const long qs = proj_stride ? proj_stride : (long)n_heads * 2 * head_dim;
    const long ks = proj_stride ? proj_stride : (long)n_kv_heads * head_dim;
    const int cap = cache_capacity, start0 = *cache_start, len0 = *cache_len;
    ANELM_REQUIRE(cap >= 1 && len0 >= 0 && len0 <= cap && start0 >= 0 && start0 < cap && pos0 >= 0,
                  "full_attn_prefill: ring start %d len %d capacity %d, position %d", start0, len0, cap, pos0);
    const long L = (long)len0 + S;
    const int D = head_dim;
    ANELM_REQUIRE(L * n_kv_heads * D * 2 < 0x7fffffffL && (long)S * n_heads * D * 2 < 0x7fffffffL,
                  "full_attn_prefill: %ld keys exceed the 2 GiB buffer range", L);
    hipStream_t st = as_stream(stream);
    const size_t qb = ((size_t)S * n_heads * D * 2 + 255) & ~(size_t)255;
    const size_t kb = ((size_t)L * n_kv_heads * D * 2 + 255) & ~(size_t)255;
    char* ws = static_cast<char*>(workspace2(qb + 2 * kb, st));
    if (!ws) return ANELM_ENOMEM;
    uint16_t* qh = reinterpret_cast<uint16_t*>(ws);
    uint16_t* kall = reinterpret_cast<uint16_t*>(ws + qb);
    uint16_t* vall = reinterpret_cast<uint16_t*>(ws + qb + kb);
    const int row16 = n_kv_heads * D / 8;
    if (len0 > 0) {
        const long n16 = (long)len0 * row16;
        hipLaunchKernelGGL(ring_gather_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, kall, vall,
                           k_cache, v_cache, n16, row16, start0, cap);
        ANELM_LAUNCHED("ring_gather_kernel");
    }
    PrepArgs a{q_gate, k, v, qs, ks, q_norm_w, k_norm_w, rope_table, rope_table ? rope_rows : 0, qh, kall, vall,
               S, n_heads, n_kv_heads, len0, pos0, rot_dim / 2, rope_mode, theta, eps};
    const dim3 pg(S, (n_heads + n_kv_heads + kPrepRowsPerWg - 1) / kPrepRowsPerWg);
    if (D == 256) hipLaunchKernelGGL(prefill_prep_kernel<256>, pg, dim3(64 * kPrepRowsPerWg), 0, st, a);
    else hipLaunchKernelGGL(prefill_prep_kernel<128>, pg, dim3(64 * kPrepRowsPerWg), 0, st, a);
    ANELM_LAUNCHED("prefill_prep_kernel");
    // rows whose ring overflowed inside the prompt see the last `cap` keys
    const int win = L > cap ? cap : 0;
    int rc = prefill_core(out, false, qh, kall, vall, S, (int)L, len0, win, n_heads, n_kv_heads, D,
                          gate ? q_gate + D : nullptr, (int)qs, 2 * D, st);
    if (rc) return rc;
    const int t0 = S > cap ? S - cap : 0;
    const long n16 = (long)(S - t0) * row16;
    hipLaunchKernelGGL(ring_write_kernel, dim3((unsigned)((n16 + 255) / 256)), dim3(256), 0, st, k_cache, v_cache,
                       kall, vall, n16, row16, t0, len0, start0, cap);
    ANELM_LAUNCHED("ring_write_kernel");
    if (L <= cap) {
        *cache_len = (int)L;
    } else {
        *cache_len = cap;
        *cache_start = (int)((start0 + L - cap) % cap);
    }
    return ANELM_OK;
}

extern "C" int anelm_deltanet_prefill_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                                                const float* proj, const float* conv_w, const float* A,
                                                const float* dt_bias, const float* norm_w, int S, int Hk, int Hv,
                                                int dk, int dv, int conv_kernel, int flags, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(state);
    ANELM_NONNULL(conv_state);
    ANELM_NONNULL(conv_pos);
    ANELM_NONNULL(proj);
    ANELM_NONNULL(conv_w);
    ANELM_NONNULL(A);
    ANELM_NONNULL(dt_bias);
    ANELM_REQUIRE(S >= 1, "deltanet_prefill_from_proj: S %d", S);
    ANELM_REQUIRE(dk == 128 && dv == 128, "deltanet_prefill_from_proj: dk=%d dv=%d (only 128x128)", dk, dv);
    ANELM_REQUIRE(Hk > 0 && Hv > 0 && Hv % Hk == 0, "deltanet_prefill_from_proj: Hv %d not a multiple of Hk %d", Hv,
                  Hk);
    ANELM_REQUIRE(conv_kernel >= 2 && conv_kernel <= 16, "deltanet_prefill_from_proj: conv kernel %d", conv_kernel);
    ANELM_REQUIRE(*conv_pos >= 0 && *conv_pos < conv_kernel - 1, "deltanet_prefill_from_proj: conv_pos %d",
                  *conv_pos);
    ANELM_REQUIRE((flags & ~7) == 0, "deltanet_prefill_from_proj: unknown flags 0x%x", flags);
    const bool gated = (flags & ANELM_DN_GATED_NORM) != 0;
    ANELM_REQUIRE(!gated || norm_w != nullptr, "deltanet_prefill_from_proj: GATED_NORM needs norm_w");
    const int nqk = Hk * dk, C = 2 * nqk + Hv * dv, nz = Hv * dv, pd = C + nz + 2 * Hv;
    ANELM_REQUIRE((long)S * pd < 0x7fffffffL, "deltanet_prefill_from_proj: %d tokens too many", S);
    hipStream_t st = as_stream(stream);
    // q, k [S][nqk]; v, z, y [S][nz]; a, b [S][Hv] -- apart from the chunked
    // prefill's own workspace
    const size_t f = sizeof(float);
    const size_t nq = (size_t)S * nqk, nv = (size_t)S * nz, na = ((size_t)S * Hv + 63) & ~(size_t)63;
    float* ws = static_cast<float*>(workspace2(f * (2 * nq + 3 * nv + 2 * na), st));
    if (!ws) return ANELM_ENOMEM;
    float *q = ws, *k = q + nq, *v = k + nq, *z = v + nv, *yr = z + nv, *a = yr + nv, *b = a + na;
    ConvArgs p{proj, conv_state, conv_w, q, k, v, z, a, b, S, C, pd, *conv_pos, nqk, nz, Hv, 64};
    const dim3 grid((C + nz + 2 * Hv + 255) / 256, (S + p.tpb - 1) / p.tpb);
    switch (conv_kernel) {
#define ANELM_CONV_CASE(KK) \
    case KK: hipLaunchKernelGGL(dn_conv_prefill_kernel<KK>, grid, dim3(256), 0, st, p); break;
        ANELM_CONV_CASE(2) ANELM_CONV_CASE(3) ANELM_CONV_CASE(4) ANELM_CONV_CASE(5) ANELM_CONV_CASE(6)
        ANELM_CONV_CASE(7) ANELM_CONV_CASE(8) ANELM_CONV_CASE(9) ANELM_CONV_CASE(10) ANELM_CONV_CASE(11)
        ANELM_CONV_CASE(12) ANELM_CONV_CASE(13) ANELM_CONV_CASE(14) ANELM_CONV_CASE(15) ANELM_CONV_CASE(16)
#undef ANELM_CONV_CASE
    }
    ANELM_LAUNCHED("dn_conv_prefill_kernel");
    hipLaunchKernelGGL(dn_conv_ring_kernel, dim3((C + 255) / 256), dim3(256), 0, st, conv_state, proj, S, C, pd,
                       conv_kernel, *conv_pos);
    ANELM_LAUNCHED("dn_conv_ring_kernel");
    int rc = anelm_deltanet_prefill(gated ? yr : y, state, q, k, v, a, b, A, dt_bias, S, Hk, Hv, dk, dv, 64,
                                    flags & 3, stream);
    if (rc) return rc;
    if (gated) {
        rc = anelm_rmsnorm_gated(y, yr, z, norm_w, dv, S * Hv, stream);
        if (rc) return rc;
    }
    *conv_pos = (int)((*conv_pos + (long)S) % (conv_kernel - 1));
    return ANELM_OK;
}
