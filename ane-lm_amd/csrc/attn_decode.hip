// Decode attention over a ring KV cache (fp16 or fp32), optionally fused with
// the q/k RMSNorm + RoPE + ring append prologue and the sigmoid output gate.
//
// Reference semantics: core/cpu_ops.cpp:148-204 (gqa_attention) composed as in
// models/llm/qwen3_5.cpp:944-1002.  The reference walks q heads one at a time
// and re-reads K/V per q head; here one workgroup owns (kv head, key split) and
// scores all G = Hq/Hkv query heads of that kv head against each K/V row read
// once.  Splits are merged with the standard (max, sum, unnormalised output)
// log-sum-exp combine: for up to 16 splits of a ring by the last workgroup of
// each kv head to finish (records handed over with device-coherent stores and
// loads, an arrival counter per kv head), else in a second small kernel.
#include "anelm_internal.hpp"

#include <type_traits>

#include <algorithm>
#include <math.h>
#include <vector>

namespace anelm {

namespace {

constexpr int kNT = 256;      // threads per workgroup
constexpr int kNW = kNT / 64;  // waves per workgroup

struct DecodeParams {
    float* out;
    const float* q;
    int q_stride;
    const void* k_cache;
    const void* v_cache;
    int n_kv_heads;
    int start, len, cap;       // ring mode
    // ring mode: element offsets of consecutive slots and of consecutive kv
    // heads -- token-major [cap][Hkv][D] (Hkv*D, D) or head-major
    // [Hkv][cap][D] (D, cap*D)
    long tok_stride, head_stride;
    float scale;
    int kps, max_splits;
    float* part;       // partials [seq][Hkv][max_splits][G][D+2]: m, l, o[D]
    uint32_t* arrivals;   // ring mode, in-kernel merge: per-kv-head arrival counters (zero); else null
    // paged mode: pages [page][Hkv][page_size][D]; key t of sequence s is
    // row t % page_size of page page_table[s*max_pages + t/page_size]
    int paged;
    const int32_t* page_table;
    const int32_t* seq_lens;
    int max_pages, page_size, n_pages, n_seqs;
    // fused prologue (ring mode only)
    int fused;
    const float* q_norm_w;
    const float* k_norm_w;
    const float* k_new;
    const float* v_new;
    void* k_cache_w;
    void* v_cache_w;
    int new_slot;
    float eps;
    int rot_pairs, rope_mode, gate;
    float cs[kMaxRotPairs];
    float sn[kMaxRotPairs];
    // fused paged step: the new token of sequence s is key seq_lens[s] at
    // position positions[s] (NULL: seq_lens[s]); RoPE rows from rope_tab
    // [rope_rows][2 * rot_pairs] (cos then sin) or, past the table, from the
    // same formula evaluated on the device
    const int32_t* positions;
    const float* rope_tab;
    int rope_rows;
    float theta;
    // paged: the q rows after the prologue kernel, fp16 [seq][Hkv][G][D]
    const uint16_t* q_prep;
};

template <typename KV> struct Raw8;
template <> struct Raw8<uint16_t> { uint4 a; };
template <> struct Raw8<float> { float4 a, b; };

__device__ __forceinline__ Raw8<uint16_t> load_raw(const uint16_t* p) {
    Raw8<uint16_t> r;
    r.a = *reinterpret_cast<const uint4*>(p);
    return r;
}
__device__ __forceinline__ Raw8<float> load_raw(const float* p) {
    Raw8<float> r;
    r.a = reinterpret_cast<const float4*>(p)[0];
    r.b = reinterpret_cast<const float4*>(p)[1];
    return r;
}
__device__ __forceinline__ void to_f32(const Raw8<uint16_t>& r, float (&f)[8]) {
    const uint32_t w[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        f[2 * i] = h2f((uint16_t)(w[i] & 0xffffu));
        f[2 * i + 1] = h2f((uint16_t)(w[i] >> 16));
    }
}
__device__ __forceinline__ void to_f32(const Raw8<float>& r, float (&f)[8]) {
    f[0] = r.a.x; f[1] = r.a.y; f[2] = r.a.z; f[3] = r.a.w;
    f[4] = r.b.x; f[5] = r.b.y; f[6] = r.b.z; f[7] = r.b.w;
}

template <typename KV> __device__ __forceinline__ Raw8<KV> make_raw(const float* v);
template <> __device__ __forceinline__ Raw8<uint16_t> make_raw<uint16_t>(const float* v) {
    Raw8<uint16_t> r;
    r.a.x = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
    r.a.y = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
    r.a.z = (uint32_t)f2h(v[4]) | ((uint32_t)f2h(v[5]) << 16);
    r.a.w = (uint32_t)f2h(v[6]) | ((uint32_t)f2h(v[7]) << 16);
    return r;
}
template <> __device__ __forceinline__ Raw8<float> make_raw<float>(const float* v) {
    Raw8<float> r;
    r.a = make_float4(v[0], v[1], v[2], v[3]);
    r.b = make_float4(v[4], v[5], v[6], v[7]);
    return r;
}

__device__ __forceinline__ void store_kv(uint16_t* p, float v) { *p = f2h(v); }
__device__ __forceinline__ void store_kv(float* p, float v) { *p = v; }

// RMSNorm (cpu_ops.cpp:24-30) + RoPE (cpu_ops.cpp:40-63) of one D-vector held
// in shared memory, in place.  All threads participate.
// A NULL weight skips the norm (callers whose q/k arrive normalised).
template <int D>
__device__ void norm_rope_row(float* row, const float* w, const DecodeParams& p, float* red, const float* cs,
                              const float* sn) {
    if (w != nullptr) {
        float ss = 0.f;
        for (int d = threadIdx.x; d < D; d += kNT) ss += row[d] * row[d];
        ss = block_sum<kNT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
        for (int d = threadIdx.x; d < D; d += kNT) row[d] = (row[d] * inv) * w[d];
    }
    __syncthreads();
    for (int j = threadIdx.x; j < p.rot_pairs; j += kNT) {
        const int i0 = p.rope_mode == 0 ? 2 * j : j;
        const int i1 = p.rope_mode == 0 ? 2 * j + 1 : j + p.rot_pairs;
        const float c = cs[j], s = sn[j];
        const float v0 = row[i0], v1 = row[i1];
        rotate_pair(row[i0], row[i1], v0, v1, c, s);
    }
    __syncthreads();
}

// The same for the G rows rows[0..G) at once: one reduction round for all
// the rows' sums of squares (partial sums in the same order as block_sum, so
// every row is normalised bit-identically to norm_rope_row).
template <int D, int G>
__device__ void norm_rope_rows(float (*rows)[D], const float* w, const DecodeParams& p, float (*red_g)[G],
                               const float* cs, const float* sn) {
    if (w != nullptr) {
        float ss[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float v = 0.f;
            for (int d = threadIdx.x; d < D; d += kNT) v += rows[g][d] * rows[g][d];
            ss[g] = wave_sum(v);
        }
        __syncthreads();
        if ((threadIdx.x & 63) == 0) {
#pragma unroll
            for (int g = 0; g < G; g++) red_g[threadIdx.x >> 6][g] = ss[g];
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < kNW; i++) t += red_g[i][g];
            const float inv = 1.0f / sqrtf(t / (float)D + p.eps);
            for (int d = threadIdx.x; d < D; d += kNT) rows[g][d] = (rows[g][d] * inv) * w[d];
        }
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * p.rot_pairs; e += kNT) {
        const int g = e / p.rot_pairs, j = e - g * p.rot_pairs;
        const int i0 = p.rope_mode == 0 ? 2 * j : j;
        const int i1 = p.rope_mode == 0 ? 2 * j + 1 : j + p.rot_pairs;
        const float c = cs[j], sv = sn[j];
        const float v0 = rows[g][i0], v1 = rows[g][i1];
        rotate_pair(rows[g][i0], rows[g][i1], v0, v1, c, sv);
    }
    __syncthreads();
}

// In-kernel merge of the split records (ring mode, 2..kInlineMaxSplits
// splits): each workgroup publishes its record with device-coherent stores,
// waits for them to complete, and counts its arrival on the (sequence, kv
// head) counter; the last to arrive reads every record of its kv head back
// with device-coherent loads, merges them, writes the output and resets the
// counter to zero (every counter is zero between calls).  Longer caches keep
// the merge kernel: there one workgroup would read too many records.
constexpr int kInlineMaxSplits = 16;
constexpr int kArrivalWords = 256;                       // counters: n_seqs * n_kv_heads <= 256
constexpr size_t kArrivalBytes = kArrivalWords * sizeof(uint32_t);

// Records go through a buffer resource with the device-coherent cache policy
// (sc1): plain loads and stores that pipeline, unlike atomic ones, each of
// which waits for the previous.
constexpr int kCoherent = 16;
__device__ __forceinline__ void st_coherent(__amdgpu_buffer_rsrc_t r, int idx, float v) {
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, idx * 4, 0, kCoherent);
}
__device__ __forceinline__ float ld_coherent(__amdgpu_buffer_rsrc_t r, int idx) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, idx * 4, 0, kCoherent));
}

// Ring-mode decode: one workgroup per (key split, kv head).  Every memory
// operand of the prologue (q rows, norm weights, the RoPE row, gate logits,
// the new key / value, this split's K and V rows) is requested up front, so
// the workgroup waits for one memory round trip before computing.
// Threads of a ring-decode workgroup: 8 waves for G <= 4 (each lane holds half
// the key rows of the 4-wave layout: the per-wave score and P V work halves),
// 4 waves for G = 8.
template <int G>
constexpr int ring_threads() { return G <= 4 ? 512 : 256; }

template <typename KV, int D, int G>
__global__ __launch_bounds__(ring_threads<G>()) void attn_decode_kernel(const DecodeParams p) {
    constexpr int NT = ring_threads<G>();
    constexpr int NW = NT / 64;
    constexpr int LPK = D / 8;        // lanes per key row (8 elements each)
    constexpr int KPI = 64 / LPK;     // key rows per wave instruction
    constexpr int KPB = NW * KPI;     // key rows per workgroup instruction
    constexpr int KPS = 256 / G;      // keys per split
    constexpr int KB = KPS / KPB;     // key rows per lane
    constexpr int R = KB * G;         // partial dots per lane (LPK, or LPK / 2 with 8 waves)
    constexpr int REC = D + 2;
    constexpr int NO = (G * D + NT - 1) / NT;   // output elements per thread
    static_assert(KB >= 1 && KB * KPB == KPS && (R == LPK || 2 * R == LPK), "split layout");
    static_assert(D <= NT, "one thread per head dimension");

    __shared__ float q_s[G + 1][D];   // the G query rows, then (owner) the new key row
    __shared__ float sc[G][KPS];
    __shared__ float red_o[NW][G][D];
    __shared__ float red_g[NW][G + 1];
    __shared__ float cs_s[kMaxRotPairs], sn_s[kMaxRotPairs];
    __shared__ float ml_s[kInlineMaxSplits][G][2];
    __shared__ float wl_s[kInlineMaxSplits][G];   // merge weights e^(m_s - M), zero past the last split
    __shared__ float L_s[G];
    __shared__ int last_s;

    const int split = blockIdx.x;
    const int kvh = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int sub = lane / LPK, dl = lane % LPK;
    const int len = p.len;
    float* const out = p.out + (size_t)kvh * G * D;
    if (len <= 0) {  // empty cache: zeros, as cpu_ops.cpp:152-155
        if (split == 0)
            for (int e = tid; e < G * D; e += NT) out[e] = 0.f;
        return;
    }
    const int n_splits = (len + p.kps - 1) / p.kps;
    if (split >= n_splits) return;
    const bool inline_merge = p.arrivals != nullptr;
    const bool finisher = n_splits == 1 || inline_merge;   // may write the output
    float* const part = p.part + (size_t)kvh * p.max_splits * G * REC;

    const int t0 = split * KPS;
    const int nk = min(KPS, len - t0);
    const size_t tok_stride = (size_t)p.tok_stride, head_off = (size_t)kvh * p.head_stride;
    const KV* kc = reinterpret_cast<const KV*>(p.k_cache);
    const KV* vc = reinterpret_cast<const KV*>(p.v_cache);
    const bool owner = p.fused && split == n_splits - 1;   // holds the newest key
    const float* qh = p.q + (size_t)kvh * G * p.q_stride;

    // ---- every operand requested at once.  With interleaved RoPE pairs (or
    // none) every lane takes the 8 dims dl*8 .. dl*8+7 of each q row (and of
    // the new key) itself: the row sums over the LPK lanes that hold it,
    // the pairs lie inside the lane, so norm and RoPE need no LDS and no
    // workgroup barrier.  Half-split pairs go through LDS (one thread per dim).
    const bool lane_rows = !p.fused || p.rope_mode == 0;
    const bool qnorm = p.fused && p.q_norm_w != nullptr;
    float qv[G];
    float q8[G][8], wq8[8], kn8[8], wk8[8];
    float wq = 1.f, wk = 1.f;
    float kn_reg = 0.f, vn_reg = 0.f;
    float vn8[8];
    if (lane_rows) {
        // 8 consecutive floats per lane: two 16-byte loads where the rows are
        // 16-byte aligned (the two halves of a lane's 32 bytes share lines)
        auto load8 = [](const float* src, float (&o)[8], bool al) __attribute__((always_inline)) {
            if (al) {
                const float4 lo = reinterpret_cast<const float4*>(src)[0];
                const float4 hi = reinterpret_cast<const float4*>(src)[1];
                o[0] = lo.x; o[1] = lo.y; o[2] = lo.z; o[3] = lo.w;
                o[4] = hi.x; o[5] = hi.y; o[6] = hi.z; o[7] = hi.w;
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) o[i] = src[i];
            }
        };
        auto al16 = [](const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; };
        const bool qal = al16(qh) && (p.q_stride & 3) == 0;
#pragma unroll
        for (int g = 0; g < G; g++) load8(qh + (size_t)g * p.q_stride + dl * 8, q8[g], qal);
        if (qnorm) {
            load8(p.q_norm_w + dl * 8, wq8, al16(p.q_norm_w));
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) wq8[i] = 1.f;
        }
        if (owner) {
            load8(p.k_new + (size_t)kvh * D + dl * 8, kn8, al16(p.k_new));
            if (p.k_norm_w != nullptr) {
                load8(p.k_norm_w + dl * 8, wk8, al16(p.k_norm_w));
            } else {
#pragma unroll
                for (int i = 0; i < 8; i++) wk8[i] = 1.f;
            }
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; g++) qv[g] = tid < D ? qh[(size_t)g * p.q_stride + tid] : 0.f;
        if (qnorm && tid < D) wq = p.q_norm_w[tid];
        if (owner && tid < D) {
            kn_reg = p.k_new[(size_t)kvh * D + tid];
            vn_reg = p.v_new[(size_t)kvh * D + tid];
            if (p.k_norm_w != nullptr) wk = p.k_norm_w[tid];
        }
    }
    if (owner) {
#pragma unroll
        for (int i = 0; i < 8; i++) vn8[i] = p.v_new[(size_t)kvh * D + dl * 8 + i];   // any alignment
    }
    // gate logits of this kv head's outputs (a workgroup that may write them)
    float gl[NO];
#pragma unroll
    for (int i = 0; i < NO; i++) {
        const int e = tid + i * NT, g = e / D, d = e % D;
        gl[i] = (p.gate && finisher && e < G * D) ? qh[(size_t)g * p.q_stride + D + d] : 0.f;
    }
    // cos / sin through pointers into the argument segment: indexing the
    // by-value arrays directly expands into a select over every entry
    const float* csp = p.cs;
    const float* snp = p.sn;
    if (!lane_rows && tid < p.rot_pairs) {
        cs_s[tid] = csp[tid];
        sn_s[tid] = snp[tid];
    }
    auto row_ptr = [&](const KV* base, int t) -> const KV* {
        int phys = p.start + t0 + t;
        if (phys >= p.cap) phys -= p.cap;
        return base + (size_t)phys * tok_stride + head_off + dl * 8;
    };
    Raw8<KV> rk[KB], rv[KB];
#pragma unroll
    for (int b = 0; b < KB; b++) {
        const int t = b * KPB + w * KPI + sub;
        if (t < nk) {
            rk[b] = load_raw(row_ptr(kc, t));
            rv[b] = load_raw(row_ptr(vc, t));
        }
    }

    float qr[G][8];
    if (lane_rows) {
        // ---- RMSNorm (sum over the row's LPK lanes) and interleaved RoPE in registers
        if (qnorm) {
#pragma unroll
            for (int g = 0; g < G; g++) {
                float ss = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) ss += q8[g][i] * q8[g][i];
                ss = wave_sum_from<LPK / 2>(ss);   // the LPK lanes holding the row
                const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
                for (int i = 0; i < 8; i++) q8[g][i] = (q8[g][i] * inv) * wq8[i];
            }
        }
        if (owner && p.k_norm_w != nullptr) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 8; i++) ss += kn8[i] * kn8[i];
            ss = wave_sum_from<LPK / 2>(ss);
            const float inv = 1.0f / sqrtf(ss / (float)D + p.eps);
#pragma unroll
            for (int i = 0; i < 8; i++) kn8[i] = (kn8[i] * inv) * wk8[i];
        }
        if (p.fused) {
#pragma unroll
            for (int m = 0; m < 4; m++) {
                const int j = dl * 4 + m;   // pair (2j, 2j + 1)
                if (j < p.rot_pairs) {
                    const float c = csp[j], sv = snp[j];
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        const float v0 = q8[g][2 * m], v1 = q8[g][2 * m + 1];
                        rotate_pair(q8[g][2 * m], q8[g][2 * m + 1], v0, v1, c, sv);
                    }
                    if (owner) {
                        const float v0 = kn8[2 * m], v1 = kn8[2 * m + 1];
                        rotate_pair(kn8[2 * m], kn8[2 * m + 1], v0, v1, c, sv);
                    }
                }
            }
        }
        if (owner) {
            // the fp16 append of the new key and value (one half-wave writes
            // the row), and the row as stored for the lane that scores it
            if (w == 0 && sub == 0) {
                KV* kw = reinterpret_cast<KV*>(p.k_cache_w) + (size_t)p.new_slot * tok_stride + head_off + dl * 8;
                KV* vw = reinterpret_cast<KV*>(p.v_cache_w) + (size_t)p.new_slot * tok_stride + head_off + dl * 8;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    store_kv(kw + i, kn8[i]);
                    store_kv(vw + i, vn8[i]);
                }
            }
            // The row loads above ran before the append: the newest key and
            // value come from the prologue instead, rounded as stored.
#pragma unroll
            for (int b = 0; b < KB; b++) {
                if (b * KPB + w * KPI + sub == nk - 1) {
                    rk[b] = make_raw<KV>(kn8);
                    rv[b] = make_raw<KV>(vn8);
                }
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) qr[g][i] = q8[g][i];
    } else {
        // ---- q rows (and the owner's key row): RMSNorm + RoPE in one reduction round
        if (tid < D) {
#pragma unroll
            for (int g = 0; g < G; g++) q_s[g][tid] = qv[g];
            q_s[G][tid] = kn_reg;
        }
        const int nrows = owner ? G + 1 : G;
        if (p.fused) {
            if (p.q_norm_w != nullptr) {
                // partial sums in the order of block_sum: per wave, then over the waves
                float ss[G + 1];
#pragma unroll
                for (int r = 0; r <= G; r++) {
                    const float v = tid < D ? (r < G ? qv[r] : kn_reg) : 0.f;
                    ss[r] = wave_sum(v * v);
                }
                if (lane == 0) {
#pragma unroll
                    for (int r = 0; r <= G; r++) red_g[w][r] = ss[r];
                }
                __syncthreads();
                if (tid < D) {
#pragma unroll
                    for (int r = 0; r <= G; r++) {
                        float t = 0.f;
#pragma unroll
                        for (int i = 0; i < NW; i++) t += red_g[i][r];
                        const float inv = 1.0f / sqrtf(t / (float)D + p.eps);
                        q_s[r][tid] = (q_s[r][tid] * inv) * (r < G ? wq : wk);
                    }
                }
            }
            __syncthreads();
            for (int e = tid; e < nrows * p.rot_pairs; e += NT) {
                const int r = e / p.rot_pairs, j = e - r * p.rot_pairs;
                const int i0 = p.rope_mode == 0 ? 2 * j : j;
                const int i1 = p.rope_mode == 0 ? 2 * j + 1 : j + p.rot_pairs;
                const float c = cs_s[j], sv = sn_s[j];
                const float v0 = q_s[r][i0], v1 = q_s[r][i1];
                rotate_pair(q_s[r][i0], q_s[r][i1], v0, v1, c, sv);
            }
        }
        __syncthreads();
        if (owner) {
            KV* kw = reinterpret_cast<KV*>(p.k_cache_w) + (size_t)p.new_slot * tok_stride + head_off;
            KV* vw = reinterpret_cast<KV*>(p.v_cache_w) + (size_t)p.new_slot * tok_stride + head_off;
            if (tid < D) {
                store_kv(kw + tid, q_s[G][tid]);
                store_kv(vw + tid, vn_reg);
            }
            // The row loads above ran before the append: the newest key and
            // value come from the prologue instead, rounded as stored.
#pragma unroll
            for (int b = 0; b < KB; b++) {
                if (b * KPB + w * KPI + sub == nk - 1) {
                    rk[b] = make_raw<KV>(&q_s[G][dl * 8]);
                    rv[b] = make_raw<KV>(vn8);
                }
            }
        }

#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) qr[g][i] = q_s[g][dl * 8 + i];
    }

    // ---- scores: one transpose reduction over the KB rows of each lane
    {
        float part_s[KB * G];
#pragma unroll
        for (int b = 0; b < KB; b++) {
            const int t = b * KPB + w * KPI + sub;
            float kf[8];
            to_f32(rk[b], kf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                float s = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) s = fmaf(qr[g][i], kf[i], s);
                part_s[b * G + g] = (t < nk) ? s : 0.f;
            }
        }
        if constexpr (R == LPK) {
            transpose_reduce<LPK, R>(part_s, dl);
        } else {
            // R values over 2R lanes: within each R-lane half, then across the halves
            transpose_reduce<R, R>(part_s, dl % R);
            part_s[0] += shfl_xor(part_s[0], R);
        }
        const int b = (dl % R) / G, g = dl % G;
        const int t = b * KPB + w * KPI + sub;
        if (t < nk && dl < R) sc[g][t] = part_s[0] * p.scale;
    }
    __syncthreads();

    // ---- softmax statistics per head over this split
    float mloc[G], lloc[G];
    if constexpr (KPS <= 64) {
        // a head's KPS scores lie in one group of KPS lanes: thread tid holds
        // key tid % KPS of head tid / KPS, reduced within its group
        // (threads past G * KPS hold no score)
        const bool own = tid < G * KPS;
        const int gg = own ? tid / KPS : 0, t = tid % KPS;
        const bool hit = own && t < nk;
        const float sv = hit ? sc[gg][t] : -INFINITY;
        const float m = wave_max_from<KPS / 2>(sv);
        const float e = hit ? __expf(sv - m) : 0.f;
        const float l = wave_sum_from<KPS / 2>(e);
        if (hit) sc[gg][t] = e;
        if (own && t == 0) { ml_s[0][gg][0] = m; ml_s[0][gg][1] = l; }
        __syncthreads();   // (also publishes the probabilities in sc)
#pragma unroll
        for (int g = 0; g < G; g++) { mloc[g] = ml_s[0][g][0]; lloc[g] = ml_s[0][g][1]; }
        __syncthreads();   // ml_s is rewritten by the merge
    } else {
        // one reduction round for all G heads each over the waves
        float mw[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float m = -INFINITY;
            for (int t = tid; t < nk; t += NT) m = fmaxf(m, sc[g][t]);
            mw[g] = wave_max(m);
        }
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < G; g++) red_g[w][g] = mw[g];
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++) {
            float t = red_g[0][g];
#pragma unroll
            for (int i = 1; i < NW; i++) t = fmaxf(t, red_g[i][g]);
            mloc[g] = t;
        }
        __syncthreads();   // red_g is rewritten below
        float lw[G];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float l = 0.f;
            for (int t = tid; t < nk; t += NT) {
                const float e = __expf(sc[g][t] - mloc[g]);
                sc[g][t] = e;
                l += e;
            }
            lw[g] = wave_sum(l);
        }
        if (lane == 0) {
#pragma unroll
            for (int g = 0; g < G; g++) red_g[w][g] = lw[g];
        }
        __syncthreads();   // (also publishes the probabilities in sc)
#pragma unroll
        for (int g = 0; g < G; g++) {
            float t = 0.f;
#pragma unroll
            for (int i = 0; i < NW; i++) t += red_g[i][g];
            lloc[g] = t;
        }
    }

    // ---- P V
    float acc[G][8];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < 8; i++) acc[g][i] = 0.f;
#pragma unroll
    for (int b = 0; b < KB; b++) {
        const int t = b * KPB + w * KPI + sub;
        if (t < nk) {
            float vf[8];
            to_f32(rv[b], vf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pg = sc[g][t];
#pragma unroll
                for (int i = 0; i < 8; i++) acc[g][i] = fmaf(pg, vf[i], acc[g][i]);
            }
        }
    }
#pragma unroll
    for (int m = LPK; m < 64; m <<= 1)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) acc[g][i] += shfl_xor(acc[g][i], m);
    if (sub == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) red_o[w][g][dl * 8 + i] = acc[g][i];
    }
    __syncthreads();

    // ---- output: direct when there is one split, else a record (+ merge)
    if (n_splits == 1) {
#pragma unroll
        for (int i = 0; i < NO; i++) {
            const int e = tid + i * NT;
            if (e >= G * D) break;
            const int g = e / D, d = e % D;
            float o = 0.f;
#pragma unroll
            for (int ww = 0; ww < NW; ww++) o += red_o[ww][g][d];
            float y = o / lloc[g];
            if (p.gate) y = y / (1.0f + expf(-gl[i]));
            out[e] = y;
        }
        return;
    }
    float* rec = part + (size_t)split * G * REC;
    // this kv head's records (n_splits of them), device-coherent
    const __amdgpu_buffer_rsrc_t rr = __builtin_amdgcn_make_buffer_rsrc(part, 0, n_splits * G * REC * 4, 0x00020000);
    for (int e = tid; e < G * D; e += NT) {
        const int g = e / D, d = e % D;
        float o = 0.f;
#pragma unroll
        for (int ww = 0; ww < NW; ww++) o += red_o[ww][g][d];
        if (inline_merge) {
            const int ri = (split * G + g) * REC;
            st_coherent(rr, ri + 2 + d, o);
            if (d == 0) {
                st_coherent(rr, ri, mloc[g]);
                st_coherent(rr, ri + 1, lloc[g]);
            }
        } else {
            rec[(size_t)g * REC + 2 + d] = o;
            if (d == 0) { rec[(size_t)g * REC] = mloc[g]; rec[(size_t)g * REC + 1] = lloc[g]; }
        }
    }
    if (!inline_merge) return;
    __builtin_amdgcn_s_waitcnt(0x0F70);   // this thread's record stores completed
    __syncthreads();
    uint32_t* const ctr = p.arrivals + kvh;
    if (tid == 0) last_s = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                           (uint32_t)(n_splits - 1);
    __syncthreads();
    if (!last_s) return;
    if (tid == 0) __hip_atomic_store(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    // ---- merge: M = max m_s, L = sum l_s e^(m_s-M), O = sum o_s e^(m_s-M),
    // out = O / L, then the sigmoid gate; every record load is issued before
    // the first is used (one memory round trip)
    float ov[NO][kInlineMaxSplits];
#pragma unroll
    for (int i = 0; i < NO; i++) {
        const int e = tid + i * NT, g = (e / D) % G, d = e % D;
#pragma unroll
        for (int sp = 0; sp < kInlineMaxSplits; sp++)
            ov[i][sp] = ld_coherent(rr, (sp * G + g) * REC + 2 + d);   // past the last split: 0 (buffer range)
    }
    if (tid < n_splits * G) {
        const int sp = tid / G, g = tid % G;
        ml_s[sp][g][0] = ld_coherent(rr, (sp * G + g) * REC);
        ml_s[sp][g][1] = ld_coherent(rr, (sp * G + g) * REC + 1);
    }
    __syncthreads();
    // one weight per (split, head), zero past the last split
    if (tid < kInlineMaxSplits * G) {
        const int sp = tid / G, g = tid % G;
        float wt = 0.f;
        if (sp < n_splits) {
            float M = -INFINITY;
            for (int s2 = 0; s2 < n_splits; s2++) M = fmaxf(M, ml_s[s2][g][0]);
            wt = __expf(ml_s[sp][g][0] - M);
        }
        wl_s[sp][g] = wt;
    }
    __syncthreads();
    if (tid < G) {
        float L = 0.f;
        for (int sp = 0; sp < n_splits; sp++) L += ml_s[sp][tid][1] * wl_s[sp][tid];
        L_s[tid] = L;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < NO; i++) {
        const int e = tid + i * NT;
        if (e >= G * D) break;
        const int g = e / D;
        float O = 0.f;
#pragma unroll
        for (int sp = 0; sp < kInlineMaxSplits; sp++) O = fmaf(wl_s[sp][g], ov[i][sp], O);
        const float L = L_s[g];
        float y = O / L;
        if (p.gate) y = y / (1.0f + expf(-gl[i]));
        out[e] = y;
    }
}

// ---- paged decode on the matrix cores (fp16 pages)
//
// A workgroup owns kPagedSplit keys of one (sequence, kv head); each of its 4
// waves walks its own 16-key blocks (block b of the split goes to wave b % 4)
// with its own online softmax, and the waves merge by log-sum-exp at the end.
// Per block, with lane l = 16 q + n:
//   S^T = K Q^T   v_mfma_f32_16x16x32_f16 over D/32 steps: A = K rows (lane
//                 holds key n, dims 32 s + 8 q .. +8), B = Q^T (lane holds q
//                 head n < G, the same dims; zero columns for n >= G).  Lane
//                 (q, n) ends with the scores of head n for keys 4 q .. 4 q + 3.
//   softmax       per head column: running maximum over the four lanes of the
//                 column, weights rounded to fp16 -- already the A operand of
//                 P V (lane (q, n) holds P[head n][keys 4 q .. 4 q + 3]).
//   O += P V      v_mfma_f32_16x16x16f16 per 16-dim tile t: B = V[keys 4 q ..
//                 4 q + 3][dim 16 t + n], read from the wave's LDS copy of the
//                 block's V rows with ds_read_b64_tr_b16 (a 16-lane group whose
//                 lanes address 4 keys x 16 dims, 8 bytes each, receives the
//                 4 x 16 block transposed: lane n gets dim n of the 4 keys).
// The V rows reach LDS by direct global-to-LDS loads (16 bytes per lane:
// key n, dims 8 (4 i + q) .. +8 of instruction i land at byte (16 (4 i + q) +
// n) * 16 of the wave's block), the K rows go to registers; both are issued
// together, K first.  Output rows of heads >= G are computed and dropped.
constexpr int kPagedSplit = 256;   // keys per workgroup
constexpr int kPagedBlk = 16;      // keys per wave block

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_void_ptr;

// cos / sin of RoPE pair j at position pos: the table row, or past the table
// the formula of cpu_ops.cpp:51-55
__device__ __forceinline__ void rope_cs(const DecodeParams& p, int pos, bool in_tab, int j, float& c, float& s) {
    const int R = p.rot_pairs;
    if (in_tab) {
        c = p.rope_tab[(size_t)pos * 2 * R + j];
        s = p.rope_tab[(size_t)pos * 2 * R + R + j];
    } else {
        const float freq = 1.0f / powf(p.theta, (float)(2 * j) / (float)(2 * R));
        const float angle = (float)pos * freq;
        c = cosf(angle);
        s = sinf(angle);
    }
}

// Inclusive prefix sum of v over the workgroup's kNT threads through s[kNT]
// (s[kNT - 1] then holds the total; every thread's s reads are done before
// the next call writes s).
__device__ int block_scan_int(int v, int* s) {
    const int tid = threadIdx.x;
    __syncthreads();
    s[tid] = v;
    __syncthreads();
    for (int off = 1; off < kNT; off <<= 1) {
        const int a = tid >= off ? s[tid - off] : 0;
        __syncthreads();
        s[tid] += a;
        __syncthreads();
    }
    return s[tid];
}

// Paged-step prologue, one workgroup per (kv head, sequence): the G q rows
// normalised and rotated (models/llm/qwen3_5.cpp:952-986 for the sequence:
// q/k RMSNorm, RoPE at its position -- the table row, or past the table the
// formula of cpu_ops.cpp:51-55), stored as fp16 for the attention kernel;
// fused, also the new key (normalised, rotated) and value appended to their
// pages as fp16.  Unfused: the q rows converted as given.
template <int D, int G>
__global__ __launch_bounds__(kNT) void attn_paged_prep_kernel(const DecodeParams p, uint16_t* qh) {
    __shared__ float q_s[G + 1][D];   // the q rows, then the new key
    __shared__ float red_g[kNW][G];
    __shared__ float red[kNW];
    __shared__ float rope_s[2][kMaxRotPairs];
    const int kvh = blockIdx.x, seq = blockIdx.y, tid = threadIdx.x;
    const int Hkv = p.n_kv_heads;
    const float* qk = p.q + ((size_t)seq * Hkv + kvh) * G * p.q_stride;
    uint16_t* const dst = qh + ((size_t)seq * Hkv + kvh) * G * D;
    for (int e = tid; e < G * D; e += kNT) q_s[e / D][e % D] = qk[(size_t)(e / D) * p.q_stride + e % D];
    if (!p.fused) {
        __syncthreads();
        for (int e = tid; e < G * D; e += kNT) dst[e] = f2h(q_s[e / D][e % D]);
        return;
    }
    const int cached = p.seq_lens[seq];
    const bool append = cached >= 0 && cached < p.len;   // the new key is attended (and stored)
    const int pos = p.positions ? p.positions[seq] : cached;
    const bool in_tab = p.rope_tab != nullptr && pos >= 0 && pos < p.rope_rows;
    for (int j = tid; j < p.rot_pairs; j += kNT) rope_cs(p, pos, in_tab, j, rope_s[0][j], rope_s[1][j]);
    __syncthreads();
    norm_rope_rows<D, G>(q_s, p.q_norm_w, p, red_g, rope_s[0], rope_s[1]);
    for (int e = tid; e < G * D; e += kNT) dst[e] = f2h(q_s[e / D][e % D]);
    if (!append) return;   // (uniform)
    const size_t nrow = ((size_t)seq * Hkv + kvh) * D;
    for (int d = tid; d < D; d += kNT) q_s[G][d] = p.k_new[nrow + d];
    __syncthreads();
    norm_rope_row<D>(q_s[G], p.k_norm_w, p, red, rope_s[0], rope_s[1]);
    const int ps = p.page_size;
    const int page = min(max(p.page_table[(size_t)seq * p.max_pages + cached / ps], 0), p.n_pages - 1);
    const size_t off = (((size_t)page * Hkv + kvh) * ps + cached % ps) * D;
    uint16_t* const kw = reinterpret_cast<uint16_t*>(p.k_cache_w) + off;
    uint16_t* const vw = reinterpret_cast<uint16_t*>(p.v_cache_w) + off;
    for (int d = tid; d < D; d += kNT) {
        kw[d] = f2h(q_s[G][d]);
        vw[d] = f2h(p.v_new[nrow + d]);
    }
}

template <int D, int G>
__global__ __launch_bounds__(kNT) __attribute__((amdgpu_waves_per_eu(3))) void attn_paged_mfma_kernel(const DecodeParams p) {
    constexpr int KS = D / 32;                // QK steps of 32 dims (also V load instructions)
    constexpr int NTD = D / 16;               // P V tiles of 16 dims
    constexpr int VB = kPagedBlk * D * 2;     // bytes of a wave's V block
    constexpr int KPS = kPagedSplit;
    constexpr int REC = D + 2;
    static_assert(G <= 8 && KS >= 2, "heads per kv head <= 8, head_dim >= 64");
    static_assert(G * D * 4 <= VB, "O rows fit in the wave's block");
    // per wave: the V block; after a run's blocks, the wave's O rows [G][D]
    __shared__ __attribute__((aligned(16))) char vblk[kNW][VB];
    __shared__ float red_g[kNW][G];
    __shared__ float red_m[kNW][G];
    __shared__ int scan_s[kNT];

    const int Hkv = p.n_kv_heads;
    const int tid = threadIdx.x;
    const int w = tid >> 6;
    const int NWG = gridDim.x, wg = blockIdx.x;
    // keys of sequence s: its cached keys, and (fused) the new one
    auto seq_len = [&](int s) {
        const int c = p.seq_lens[s];
        return p.fused ? min(c + 1, p.len) : min(c, p.len);
    };
    auto units_of = [&](int L) { return L > 0 ? Hkv * ((L + KPS - 1) / KPS) : 0; };

    // ---- this workgroup's units: the (sequence, kv head, split) units in
    // sequence-major order, U in all, split evenly over the NWG workgroups
    // (every workgroup scans the lengths; empty sequences get zeros here)
    int U = 0;
    for (int c0 = 0; c0 < p.n_seqs; c0 += kNT) {
        const int s = c0 + tid;
        block_scan_int(s < p.n_seqs ? units_of(seq_len(s)) : 0, scan_s);
        U += scan_s[kNT - 1];
    }
    for (int s = wg; s < p.n_seqs; s += NWG) {   // empty sequences: zeros, as cpu_ops.cpp:152-155
        if (seq_len(s) > 0) continue;
        float* o0 = p.out + (size_t)s * Hkv * G * D;
        for (int e = tid; e < Hkv * G * D; e += kNT) o0[e] = 0.f;
    }
    const int u0 = (int)(((long long)U * wg) / NWG), u1 = (int)(((long long)U * (wg + 1)) / NWG);
    if (u0 >= u1) return;   // (uniform)
    // the sequence holding unit u0 and the units before it
    int seq = 0, ubase = 0;
    for (int c0 = 0; c0 < p.n_seqs; c0 += kNT) {
        const int s = c0 + tid;
        const int us = s < p.n_seqs ? units_of(seq_len(s)) : 0;
        const int incl = block_scan_int(us, scan_s);   // inclusive, chunk-local
        const int total = scan_s[kNT - 1];
        // the thread whose range [ubase + incl - us, ubase + incl) holds u0
        const int lo = ubase + incl - us;
        __syncthreads();
        if (s < p.n_seqs && us > 0 && u0 >= lo && u0 < lo + us) scan_s[0] = s, scan_s[1] = lo;
        __syncthreads();
        const bool found = u0 < ubase + total;
        if (found) {
            seq = scan_s[0];
            ubase = scan_s[1];
        }
        __syncthreads();
        if (found) break;
        ubase += total;
    }

    const uint16_t* kc = reinterpret_cast<const uint16_t*>(p.k_cache);
    const uint16_t* vc = reinterpret_cast<const uint16_t*>(p.v_cache);
    const int ps = p.page_size;
    const unsigned rows_per_page = (unsigned)(Hkv * ps);
    char* const vb = vblk[w];

    // ---- runs: the units of one (sequence, kv head) taken together, keys
    // [s0 KPS, min((s1 + 1) KPS, L)) with one online softmax
    int u = u0;
    while (u < u1) {
        // lane quantities are derived here, per run, not held across runs
        int lane = tid & 63;
        asm volatile("" : "+v"(lane));
        const int q = lane >> 4, n = lane & 15;
        // transposed reads: lane n of group q addresses key 4 q + n/4, dims
        // 16 t + 4 (n % 4) .. +4 of tile t
        const int tr_off = (16 * ((n & 3) >> 1) + 4 * q + (n >> 2)) * 16 + (n & 1) * 8;
        const int L = seq_len(seq);
        const int ns = L > 0 ? (L + KPS - 1) / KPS : 0;
        if (u >= ubase + Hkv * ns) {   // (uniform) next sequence
            ubase += Hkv * ns;
            seq++;
            continue;
        }
        const int local = u - ubase, kvh = local / ns, s0 = local - kvh * ns;
        const int s1 = min(ns - 1, s0 + (u1 - u) - 1);
        u += s1 - s0 + 1;
        const int k0 = s0 * KPS, kend = min((s1 + 1) * KPS, L), nk_all = kend - k0;
        const unsigned k_last = (unsigned)(kend - 1);
        const int nblk = (nk_all + kPagedBlk - 1) / kPagedBlk;
        const float* qseq = p.q + (size_t)seq * Hkv * G * p.q_stride;
        const int32_t* ptab = p.page_table + (size_t)seq * p.max_pages;
        const unsigned head_row = (unsigned)(kvh * ps);

        // q (normalised, rotated, fp16: the prologue kernel's rows) as the B
        // operand of S^T = K Q^T: lane (q, n) holds head n, dims 32 s + 8 q
        // .. +8 (zero columns past the G heads)
        const uint16_t* qrow = p.q_prep + (((size_t)seq * Hkv + kvh) * G + min(n, G - 1)) * D;
        half8_t qb[KS];
#pragma unroll
        for (int s = 0; s < KS; s++) {
            qb[s] = *reinterpret_cast<const half8_t*>(qrow + 32 * s + 8 * q);
            if (n >= G) qb[s] = half8_t{};
        }

        // ---- the run's 16-key blocks, block b to wave b % 4; key n of a
        // block (past the run's last key: that key again, masked) through its
        // page-table entry, the next block's entry requested a block ahead
        f32x4_t o[NTD];
#pragma unroll
        for (int t = 0; t < NTD; t++) o[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
        float m_run = -INFINITY, l_run = 0.f;   // head n of this wave
        auto key_of = [&](int blk) { return min((unsigned)(k0 + blk * kPagedBlk + n), k_last); };
        auto entry = [&](unsigned kt) { return ptab[kt / (unsigned)ps]; };
        int pe = entry(key_of(w));
        for (int blk = w; blk < nblk; blk += kNW) {
            const unsigned kt = key_of(blk);
            const unsigned pi = kt / (unsigned)ps;
            const unsigned page = (unsigned)min(max(pe, 0), p.n_pages - 1);
            const size_t base = (size_t)(page * rows_per_page + head_row + (kt - pi * (unsigned)ps)) * D;
            pe = entry(key_of(blk + kNW));
            half8_t ka[KS];
#pragma unroll
            for (int s = 0; s < KS; s++) ka[s] = *reinterpret_cast<const half8_t*>(kc + base + 32 * s + 8 * q);
            // the V rows straight into the wave's LDS block: key n, dims
            // 8 (4 i + q) .. +8 at byte (16 (4 i + q) + n) * 16
#pragma unroll
            for (int i = 0; i < KS; i++)
                __builtin_amdgcn_global_load_lds(vc + base + 8 * (4 * i + q), (lds_void_ptr)(vb + i * 1024), 16, 0, 0);
            f32x4_t st = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < KS; s++) st = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], qb[s], st, 0, 0, 0);
            // ---- online softmax of head n over keys 4 q + i of the block
            float sc[4], bm = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = blk * kPagedBlk + 4 * q + i;
                sc[i] = t < nk_all ? st[i] * p.scale : -INFINITY;
                bm = fmaxf(bm, sc[i]);
            }
            bm = fmaxf(bm, partner<32>(bm));
            bm = fmaxf(bm, partner<16>(bm));
            const float m_new = fmaxf(m_run, bm);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;   // no valid key yet: weights 0
            const float alpha = __expf(m_run - m_use);              // 0 while m_run is -inf
            half4_t pa;
            float psum = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float e = __expf(sc[i] - m_use);   // masked keys: 0
                psum += e;
                pa[i] = (_Float16)e;
            }
            l_run = l_run * alpha + psum;
            m_run = m_new;
            // O row 4 q + i is head 4 q + i: its factor is that column's alpha
            if (__any(n < G && alpha != 1.f)) {
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const float ai = __shfl(alpha, 4 * q + i, 64);
#pragma unroll
                    for (int t = 0; t < NTD; t++) o[t][i] *= ai;
                }
            }
            // ---- O += P V, V^T tiles from the block in LDS
#pragma unroll
            for (int t = 0; t < NTD; t++) {
                const s16x4_t vt = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (__attribute__((address_space(3))) s16x4_t*)(vb + t * 512 + tr_off));
                o[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, __builtin_bit_cast(half4_t, vt), o[t], 0, 0, 0);
            }
        }

        // ---- merge the waves: per head M = max of the waves' maxima, each
        // wave weighed by e^(m_w - M); one record for the run's first split
        // (the rest of its splits marked empty), or the output itself when
        // the sequence has one split
        float lt = l_run;
        lt += partner<32>(lt);
        lt += partner<16>(lt);
        if (lane < G) {
            red_m[w][lane] = m_run;
            red_g[w][lane] = lt;
        }
        float* ro = reinterpret_cast<float*>(vb);   // this wave's O rows [G][D]
#pragma unroll
        for (int t = 0; t < NTD; t++)
#pragma unroll
            for (int i = 0; i < 4; i++)
                if (4 * q + i < G) ro[(4 * q + i) * D + 16 * t + n] = o[t][i];
        __syncthreads();
        float mtot[G], ltot[G], wsc[G][kNW];
#pragma unroll
        for (int g = 0; g < G; g++) {
            float M = red_m[0][g];
#pragma unroll
            for (int ww = 1; ww < kNW; ww++) M = fmaxf(M, red_m[ww][g]);
            const float Mu = M == -INFINITY ? 0.f : M;
            mtot[g] = M;
            ltot[g] = 0.f;
#pragma unroll
            for (int ww = 0; ww < kNW; ww++) {
                wsc[g][ww] = __expf(red_m[ww][g] - Mu);   // a wave without valid keys: 0
                ltot[g] += red_g[ww][g] * wsc[g][ww];
            }
        }
        float* const outs = p.out + (size_t)seq * Hkv * G * D;
        float* const recs = p.part + ((size_t)seq * Hkv + kvh) * p.max_splits * G * REC;
        for (int e = tid; e < G * D; e += kNT) {
            const int g = e / D, d = e % D;
            float o2 = 0.f;
#pragma unroll
            for (int ww = 0; ww < kNW; ww++) o2 += reinterpret_cast<const float*>(vblk[ww])[e] * wsc[g][ww];
            if (ns == 1) {
                const int hq = kvh * G + g;
                float yv = o2 / ltot[g];
                if (p.gate) yv = yv / (1.0f + expf(-qseq[(size_t)hq * p.q_stride + D + d]));
                outs[(size_t)hq * D + d] = yv;
            } else {
                float* rec = recs + ((size_t)s0 * G + g) * REC;
                rec[2 + d] = o2;
                if (d == 0) {
                    rec[0] = mtot[g];
                    rec[1] = ltot[g];
                }
            }
        }
        // the run's other splits: empty records (l = 0: the merge skips them)
        for (int e = tid; e < (s1 - s0) * G; e += kNT) {
            float* rec = recs + ((size_t)(s0 + 1 + e / G) * G + e % G) * REC;
            rec[0] = -INFINITY;
            rec[1] = 0.f;
        }
        __syncthreads();   // (LDS reused by the next run)
    }
}

// Log-sum-exp merge of the split partials of one (sequence, q head) for 64
// output dims per workgroup: M = max m_s, L = sum l_s e^(m_s-M),
// O = sum o_s e^(m_s-M), out = O / L, then the sigmoid gate.  Splits are
// taken kCombineRound at a time, and every load of a round is issued before
// any of its arithmetic: thread t reads m and l of split t of the round, and
// the four groups of 64 threads read the o values of interleaved quarters of
// the round's splits (kCombineRound / 4 each, all in flight together).  The
// round's maximum and weights then go through LDS; a later round rescales the
// running sums when the maximum grows.  R splits per round (<= the 256
// threads): 128 for the ring's records, whose o values are requested with
// m and l; 64 for paged records, most of which are empty (one record per
// workgroup run): their o values are requested once the weights are known,
// only for the records that carry weight.
template <int D, int G, int R, bool PAGED>
__global__ __launch_bounds__(256) void attn_combine_kernel(const DecodeParams p) {
    constexpr int REC = D + 2, NQ = R / 4;
    __shared__ float f[R];
    __shared__ float red[4];
    __shared__ float osum[4][64];
    const int tid = threadIdx.x, dq = tid & 63, grp = tid >> 6;
    const int d = blockIdx.x * 64 + dq;
    const int h = blockIdx.y, seq = blockIdx.z;
    const int Hkv = p.n_kv_heads;
    const int kvh = h / G, g = h % G;
    const int len = p.paged ? min(p.seq_lens[seq] + (p.fused ? 1 : 0), p.len) : p.len;
    const int n = (len + p.kps - 1) / p.kps;
    if (n <= 1) return;   // written directly by the split kernel (or zeros)
    const size_t rs = (size_t)G * REC;   // record stride between splits
    const float* base = p.part + ((size_t)seq * Hkv + kvh) * p.max_splits * rs + (size_t)g * REC;
    float M = -INFINITY, L = 0.f, O = 0.f;
    for (int c0 = 0; c0 < n; c0 += R) {
        const int cn = min(R, n - c0);
        float mv = -INFINITY, lv = 0.f;
        if (tid < cn) {
            const float* r = base + (size_t)(c0 + tid) * rs;
            mv = r[0];
            lv = r[1];
        }
        float ov[NQ];
        if constexpr (!PAGED) {
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                const int sj = grp + 4 * j;
                ov[j] = sj < cn ? base[(size_t)(c0 + sj) * rs + 2 + d] : 0.f;
            }
        }
        const float Mn = fmaxf(M, block_max<256>(mv, red));
        // (an empty record, m = -inf and l = 0, weighs 0 and its o is not used)
        const float wv = mv != -INFINITY ? __expf(mv - Mn) : 0.f;
        const float sc = M != -INFINITY ? __expf(M - Mn) : 0.f;
        if (tid < R) f[tid] = wv;
        L = L * sc + block_sum<256>(tid < cn ? lv * wv : 0.f, red);   // (its barriers also publish f)
        O *= sc;
        if constexpr (PAGED) {
#pragma unroll
            for (int j = 0; j < NQ; j++) {
                const int sj = grp + 4 * j;
                ov[j] = sj < cn && f[sj] != 0.f ? base[(size_t)(c0 + sj) * rs + 2 + d] : 0.f;
            }
        }
#pragma unroll
        for (int j = 0; j < NQ; j++) {
            const int sj = grp + 4 * j;
            if (sj < cn && f[sj] != 0.f) O += f[sj] * ov[j];
        }
        M = Mn;
        __syncthreads();   // f is rewritten by the next round
    }
    osum[grp][dq] = O;
    __syncthreads();
    if (grp == 0) {
        float y = (osum[0][dq] + osum[1][dq] + osum[2][dq] + osum[3][dq]) / L;
        const float* q = p.q + (size_t)seq * Hkv * G * p.q_stride;
        if (p.gate) y = y / (1.0f + expf(-q[(size_t)h * p.q_stride + D + d]));
        p.out[((size_t)seq * Hkv * G + h) * D + d] = y;
    }
}

template <typename KV, int D, int G>
int launch_g(DecodeParams& p, dim3 grid, hipStream_t st) {
    if (p.paged) {
        if constexpr (!std::is_same<KV, uint16_t>::value || D < 64) {
            return set_error(ANELM_EINVAL, "paged decode: fp16 pages of head_dim >= 64 only");
        } else {
            // as many workgroups as are resident at once, each with an even
            // share of the units (the kernel divides them)
            static int per_cu = 0;
            if (per_cu == 0) {
                int nb = 0;
                if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, attn_paged_mfma_kernel<D, G>, kNT, 0) !=
                        hipSuccess ||
                    nb < 1)
                    nb = 1;
                per_cu = nb;
            }
            Device* dev = device();
            if (dev == nullptr) return ANELM_EHIP;
            hipLaunchKernelGGL((attn_paged_prep_kernel<D, G>), dim3(p.n_kv_heads, p.n_seqs), dim3(kNT), 0, st, p,
                               const_cast<uint16_t*>(p.q_prep));
            ANELM_LAUNCHED("attn_paged_prep_kernel");
            const dim3 pgrid(std::max(1, per_cu * dev->num_cus));
            hipLaunchKernelGGL((attn_paged_mfma_kernel<D, G>), pgrid, dim3(kNT), 0, st, p);
            ANELM_LAUNCHED("attn_paged_mfma_kernel");
        }
    } else {
        hipLaunchKernelGGL((attn_decode_kernel<KV, D, G>), grid, dim3(ring_threads<G>()), 0, st, p);
        ANELM_LAUNCHED("attn_decode_kernel");
    }
    if (p.max_splits > 1 && p.arrivals == nullptr) {
        dim3 cgrid(D / 64, grid.y * G, grid.z);
        if (p.paged)
            hipLaunchKernelGGL((attn_combine_kernel<D, G, 64, true>), cgrid, dim3(256), 0, st, p);
        else
            hipLaunchKernelGGL((attn_combine_kernel<D, G, 128, false>), cgrid, dim3(256), 0, st, p);
        ANELM_LAUNCHED("attn_combine_kernel");
    }
    return ANELM_OK;
}

template <typename KV, int D>
int launch_d(DecodeParams& p, int G, dim3 grid, hipStream_t st) {
    switch (G) {
        case 1: return launch_g<KV, D, 1>(p, grid, st);
        case 2: return launch_g<KV, D, 2>(p, grid, st);
        case 4: return launch_g<KV, D, 4>(p, grid, st);
        case 8: return launch_g<KV, D, 8>(p, grid, st);
        default: return set_error(ANELM_EINVAL, "n_heads/n_kv_heads = %d unsupported (1,2,4,8)", G);
    }
}

template <typename KV>
int launch_kv(DecodeParams& p, int D, int G, dim3 grid, hipStream_t st) {
    switch (D) {
        case 64: return (G <= 8) ? launch_d<KV, 64>(p, G, grid, st) : ANELM_EINVAL;
        case 128: return launch_d<KV, 128>(p, G, grid, st);
        case 256: return launch_d<KV, 256>(p, G, grid, st);
        default: return set_error(ANELM_EINVAL, "head_dim %d unsupported (64,128,256)", D);
    }
}

// Bytes of split partials one decode call needs (0 when one split suffices).
size_t part_bytes(int n_heads, int n_kv_heads, int D, int n_seqs, int max_len, bool paged) {
    const int G = n_heads / n_kv_heads;
    const int kps = paged ? kPagedSplit : 256 / G;
    const int max_splits = (max_len + kps - 1) / kps;
    if (max_splits <= 1) return 0;
    return (size_t)n_seqs * n_kv_heads * max_splits * G * (D + 2) * sizeof(float);
}

// Sets the split layout and partials buffer for one decode call, then
// launches.  A split is 256/G keys (ring mode: every lane of the workgroup
// then loads all of its K and V rows at once) or kPagedSplit keys (paged
// mode, 16-key blocks per wave).  `max_len` bounds every sequence's key count; `n_seqs`
// sequences (1 in ring mode).  The partials go to `part` (part_cap bytes)
// when it is given, else to the library workspace.
int run_decode(DecodeParams& p, int kv_dtype, int n_heads, int D, int n_seqs, int max_len,
               hipStream_t st, float* part = nullptr, size_t part_cap = 0) {
    const int Hkv = p.n_kv_heads;
    const int G = n_heads / Hkv;
    const int kps = p.paged ? kPagedSplit : 256 / G;
    const int max_splits = (max_len + kps - 1) / kps;
    p.kps = kps;
    p.max_splits = max_splits;
    p.n_seqs = n_seqs;
    if (p.tok_stride == 0) {   // token-major ring
        p.tok_stride = (long)Hkv * D;
        p.head_stride = D;
    }
    const size_t need = part_bytes(n_heads, Hkv, D, n_seqs, max_len, p.paged != 0);
    // ring mode with few splits: merged in the split kernel (arrival counters)
    const bool merge_inline = !p.paged && max_splits >= 2 && max_splits <= kInlineMaxSplits &&
                              Hkv * n_seqs <= kArrivalWords;
    p.arrivals = nullptr;
    if (p.paged) {
        // records, then the q rows of the paged prologue (fp16)
        const size_t rec_bytes = (need + 255) & ~(size_t)255;
        char* ws = static_cast<char*>(workspace(rec_bytes + (size_t)n_seqs * n_heads * D * 2, st));
        if (!ws) return ANELM_ENOMEM;
        p.part = need > 0 ? reinterpret_cast<float*>(ws) : nullptr;
        p.q_prep = reinterpret_cast<const uint16_t*>(ws + rec_bytes);
    } else if (need > 0 && part != nullptr) {
        // a caller's buffer holds the records from its start and, in its last
        // kArrivalBytes (zero when the caller hands it over), the counters
        if (need + (merge_inline ? kArrivalBytes : 0) > part_cap)
            return set_error(ANELM_ERANGE, "decode attention: %zu bytes of split partials, buffer holds %zu",
                             need + (merge_inline ? kArrivalBytes : 0), part_cap);
        p.part = part;
        if (merge_inline)
            p.arrivals = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(part) +
                                                     ((part_cap - kArrivalBytes) & ~(size_t)255));
    } else if (need > 0) {
        float* ws = static_cast<float*>(workspace(need, st));
        if (!ws) return ANELM_ENOMEM;
        p.part = ws;
        if (merge_inline) {
            p.arrivals = counters((size_t)Hkv * n_seqs, kCtrDecode, st);
            if (p.arrivals == nullptr) return ANELM_ENOMEM;
        }
    } else {
        p.part = nullptr;
    }
    dim3 grid(max_splits, Hkv, n_seqs);
    return kv_dtype == ANELM_F16 ? launch_kv<uint16_t>(p, D, G, grid, st)
                                 : launch_kv<float>(p, D, G, grid, st);
}

__global__ void zero_kernel(float* out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = 0.f;
}

int check_heads(int n_heads, int n_kv_heads, int head_dim) {
    ANELM_REQUIRE(n_heads > 0 && n_kv_heads > 0 && n_heads % n_kv_heads == 0,
                  "n_heads %d must be a positive multiple of n_kv_heads %d", n_heads, n_kv_heads);
    const int G = n_heads / n_kv_heads;
    ANELM_REQUIRE(G == 1 || G == 2 || G == 4 || G == 8, "n_heads/n_kv_heads = %d unsupported", G);
    ANELM_REQUIRE(head_dim == 64 || head_dim == 128 || head_dim == 256,
                  "head_dim %d unsupported (64,128,256)", head_dim);
    ANELM_REQUIRE(!(head_dim == 64 && G > 8), "head_dim 64 supports G <= 8");
    return ANELM_OK;
}

}  // namespace

}  // namespace anelm

using namespace anelm;

extern "C" int anelm_gqa_attention(float* out, const float* q, const void* k_cache,
                                   const void* v_cache, int kv_dtype, int n_heads, int n_kv_heads,
                                   int head_dim, int q_head_stride, int cache_start, int cache_len,
                                   int cache_capacity, void* stream) {
    ANELM_NONNULL(out);
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc) return rc;
    ANELM_REQUIRE(kv_dtype == ANELM_F16 || kv_dtype == ANELM_F32, "kv_dtype %d unknown", kv_dtype);
    hipStream_t st = as_stream(stream);
    if (cache_len <= 0) {
        // zeros (cpu_ops.cpp:152-155) from a fill kernel: the call stays
        // capturable into a HIP graph without a memset node
        const int n = n_heads * head_dim;
        hipLaunchKernelGGL(zero_kernel, dim3((n + 255) / 256), dim3(256), 0, st, out, n);
        ANELM_LAUNCHED("zero_kernel");
        return ANELM_OK;
    }
    ANELM_NONNULL(q);
    ANELM_NONNULL(k_cache);
    ANELM_NONNULL(v_cache);
    ANELM_REQUIRE(q_head_stride >= head_dim, "q_head_stride %d < head_dim", q_head_stride);
    ANELM_REQUIRE(cache_capacity > 0 && cache_len <= cache_capacity && cache_start >= 0 &&
                      cache_start < cache_capacity,
                  "ring (start %d, len %d, capacity %d) inconsistent", cache_start, cache_len,
                  cache_capacity);
    DecodeParams p{};
    p.out = out;
    p.q = q;
    p.q_stride = q_head_stride;
    p.k_cache = k_cache;
    p.v_cache = v_cache;
    p.n_kv_heads = n_kv_heads;
    p.start = cache_start;
    p.len = cache_len;
    p.cap = cache_capacity;
    p.scale = 1.0f / sqrtf((float)head_dim);
    p.fused = 0;
    p.gate = 0;
    return run_decode(p, kv_dtype, n_heads, head_dim, 1, cache_len, st);
}

namespace anelm {

int full_attn_decode_impl(float* out, const float* q_gate, const float* k, const float* v, uint16_t* k_cache,
                          uint16_t* v_cache, const float* q_norm_w, const float* k_norm_w, int n_heads,
                          int n_kv_heads, int head_dim, int rot_dim, int pos, float theta, float eps,
                          int rope_mode, int gate, const float* cos_row, const float* sin_row, int* cache_start,
                          int* cache_len, int cache_capacity, hipStream_t stream, float* part,
                          size_t part_cap) {
    return full_attn_decode_kv_impl(out, q_gate, k, v, k_cache, v_cache, ANELM_F16, ANELM_KV_TOKEN_MAJOR, q_norm_w,
                                    k_norm_w, n_heads, n_kv_heads, head_dim, rot_dim, pos, theta, eps, rope_mode,
                                    gate, cos_row, sin_row, cache_start, cache_len, cache_capacity, stream, part,
                                    part_cap);
}

int full_attn_decode_kv_impl(float* out, const float* q_gate, const float* k, const float* v, void* k_cache,
                             void* v_cache, int kv_dtype, int layout, const float* q_norm_w, const float* k_norm_w,
                             int n_heads, int n_kv_heads, int head_dim, int rot_dim, int pos, float theta, float eps,
                             int rope_mode, int gate, const float* cos_row, const float* sin_row, int* cache_start,
                             int* cache_len, int cache_capacity, hipStream_t stream, float* part,
                             size_t part_cap) {
    ANELM_REQUIRE(kv_dtype == ANELM_F16 || kv_dtype == ANELM_F32, "kv_dtype %d unknown", kv_dtype);
    ANELM_REQUIRE(layout == ANELM_KV_TOKEN_MAJOR || layout == ANELM_KV_HEAD_MAJOR, "cache layout %d unknown",
                  layout);
    ANELM_NONNULL(out);
    ANELM_NONNULL(q_gate);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_NONNULL(k_cache);
    ANELM_NONNULL(v_cache);
    ANELM_REQUIRE((q_norm_w == nullptr) == (k_norm_w == nullptr),
                  "q_norm_w and k_norm_w must both be given or both be NULL");
    ANELM_NONNULL(cache_start);
    ANELM_NONNULL(cache_len);
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc) return rc;
    ANELM_REQUIRE(rot_dim >= 0 && rot_dim % 2 == 0 && rot_dim <= head_dim &&
                      rot_dim / 2 <= kMaxRotPairs,
                  "rot_dim %d must be even and <= head_dim", rot_dim);
    ANELM_REQUIRE(rope_mode == ANELM_ROPE_INTERLEAVED || rope_mode == ANELM_ROPE_HALF_SPLIT,
                  "rope_mode %d unknown", rope_mode);
    ANELM_REQUIRE(cache_capacity > 0 && *cache_len >= 0 && *cache_len <= cache_capacity &&
                      *cache_start >= 0 && *cache_start < cache_capacity,
                  "ring (start %d, len %d, capacity %d) inconsistent", *cache_start, *cache_len,
                  cache_capacity);
    // Ring bookkeeping, models/llm/qwen3_5.cpp:973-983.
    int start = *cache_start, len = *cache_len, slot;
    if (len < cache_capacity) {
        slot = start + len;
        if (slot >= cache_capacity) slot -= cache_capacity;
        len++;
    } else {
        slot = start;
        start++;
        if (start >= cache_capacity) start = 0;
    }
    DecodeParams p{};
    p.out = out;
    p.q = q_gate;
    p.q_stride = 2 * head_dim;
    p.k_cache = k_cache;
    p.v_cache = v_cache;
    p.n_kv_heads = n_kv_heads;
    p.start = start;
    p.len = len;
    p.cap = cache_capacity;
    if (layout == ANELM_KV_HEAD_MAJOR) {
        p.tok_stride = head_dim;
        p.head_stride = (long)cache_capacity * head_dim;
    }
    p.scale = 1.0f / sqrtf((float)head_dim);
    p.fused = 1;
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.k_new = k;
    p.v_new = v;
    p.k_cache_w = k_cache;
    p.v_cache_w = v_cache;
    p.new_slot = slot;
    p.eps = eps;
    p.rot_pairs = rot_dim / 2;
    p.rope_mode = rope_mode;
    p.gate = gate ? 1 : 0;
    if (cos_row && sin_row) {
        for (int j = 0; j < rot_dim / 2; j++) { p.cs[j] = cos_row[j]; p.sn[j] = sin_row[j]; }
    } else {
        rope_row(p.cs, p.sn, rot_dim, pos, theta);
    }
    rc = run_decode(p, kv_dtype, n_heads, head_dim, 1, len, stream, part, part_cap);
    if (rc == ANELM_OK) {
        *cache_start = start;
        *cache_len = len;
    }
    return rc;
}

size_t full_attn_part_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len) {
    // records, plus the arrival counters at the end of a caller's buffer
    const size_t b = part_bytes(n_heads, n_kv_heads, head_dim, 1, max_len, false);
    return b > 0 ? ((b + 255) & ~(size_t)255) + kArrivalBytes : 0;
}

}  // namespace anelm

extern "C" int anelm_full_attn_decode(float* out, const float* q_gate, const float* k,
                                      const float* v, uint16_t* k_cache, uint16_t* v_cache,
                                      const float* q_norm_w, const float* k_norm_w, int n_heads,
                                      int n_kv_heads, int head_dim, int rot_dim, int pos,
                                      float theta, float eps, int rope_mode, int gate,
                                      const float* cos_row, const float* sin_row,
                                      int* cache_start, int* cache_len, int cache_capacity,
                                      void* stream) {
    return full_attn_decode_impl(out, q_gate, k, v, k_cache, v_cache, q_norm_w, k_norm_w, n_heads, n_kv_heads,
                                 head_dim, rot_dim, pos, theta, eps, rope_mode, gate, cos_row, sin_row,
                                 cache_start, cache_len, cache_capacity, as_stream(stream), nullptr, 0);
}

extern "C" int anelm_full_attn_decode_kv(float* out, const float* q_gate, const float* k, const float* v,
                                         void* k_cache, void* v_cache, int kv_dtype, int layout,
                                         const float* q_norm_w, const float* k_norm_w, int n_heads, int n_kv_heads,
                                         int head_dim, int rot_dim, int pos, float theta, float eps, int rope_mode,
                                         int gate, const float* cos_row, const float* sin_row, int* cache_start,
                                         int* cache_len, int cache_capacity, void* stream) {
    return full_attn_decode_kv_impl(out, q_gate, k, v, k_cache, v_cache, kv_dtype, layout, q_norm_w, k_norm_w,
                                    n_heads, n_kv_heads, head_dim, rot_dim, pos, theta, eps, rope_mode, gate,
                                    cos_row, sin_row, cache_start, cache_len, cache_capacity, as_stream(stream),
                                    nullptr, 0);
}

extern "C" int anelm_attn_decode_paged(float* out, const float* q, int q_head_stride,
                                       const uint16_t* k_pages, const uint16_t* v_pages,
                                       const int32_t* page_table, const int32_t* seq_lens,
                                       int n_seqs, int max_pages, int page_size, int n_pages,
                                       int max_seq_len,
                                       int n_heads, int n_kv_heads, int head_dim, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(q);
    ANELM_NONNULL(k_pages);
    ANELM_NONNULL(v_pages);
    ANELM_NONNULL(page_table);
    ANELM_NONNULL(seq_lens);
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc) return rc;
    ANELM_REQUIRE(n_seqs > 0 && n_seqs <= 65535, "paged: n_seqs %d", n_seqs);
    ANELM_REQUIRE(page_size > 0 && max_pages > 0 && n_pages > 0,
                  "paged: page_size %d max_pages %d n_pages %d", page_size, max_pages, n_pages);
    ANELM_REQUIRE((long long)n_pages * n_kv_heads * page_size < (1LL << 31),
                  "paged: %d pages of %d rows x %d kv heads exceed 2^31 cache rows", n_pages, page_size,
                  n_kv_heads);
    ANELM_REQUIRE(max_seq_len > 0 && max_seq_len <= max_pages * page_size,
                  "paged: max_seq_len %d beyond max_pages*page_size", max_seq_len);
    ANELM_REQUIRE(q_head_stride >= head_dim, "paged: q_head_stride %d < head_dim", q_head_stride);
    DecodeParams p{};
    p.out = out;
    p.q = q;
    p.q_stride = q_head_stride;
    p.k_cache = k_pages;
    p.v_cache = v_pages;
    p.n_kv_heads = n_kv_heads;
    p.scale = 1.0f / sqrtf((float)head_dim);
    p.paged = 1;
    p.page_table = page_table;
    p.seq_lens = seq_lens;
    p.max_pages = max_pages;
    p.page_size = page_size;
    p.n_pages = n_pages;
    p.len = max_seq_len;
    return run_decode(p, ANELM_F16, n_heads, head_dim, n_seqs, max_seq_len, as_stream(stream));
}

extern "C" int anelm_attn_decode_paged_step(float* out, const float* q_gate, const float* k, const float* v,
                                            uint16_t* k_pages, uint16_t* v_pages, const int32_t* page_table,
                                            const int32_t* seq_lens, const int32_t* positions,
                                            const float* q_norm_w, const float* k_norm_w,
                                            const float* rope_table, int rope_rows, int n_seqs, int max_pages,
                                            int page_size, int n_pages, int max_seq_len, int n_heads,
                                            int n_kv_heads, int head_dim, int rot_dim, float theta, float eps,
                                            int rope_mode, int gate, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(q_gate);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_NONNULL(k_pages);
    ANELM_NONNULL(v_pages);
    ANELM_NONNULL(page_table);
    ANELM_NONNULL(seq_lens);
    ANELM_REQUIRE((q_norm_w == nullptr) == (k_norm_w == nullptr),
                  "q_norm_w and k_norm_w must both be given or both be NULL");
    int rc = check_heads(n_heads, n_kv_heads, head_dim);
    if (rc) return rc;
    ANELM_REQUIRE(n_seqs > 0 && n_seqs <= 65535, "paged step: n_seqs %d", n_seqs);
    ANELM_REQUIRE(page_size > 0 && max_pages > 0 && n_pages > 0,
                  "paged step: page_size %d max_pages %d n_pages %d", page_size, max_pages, n_pages);
    ANELM_REQUIRE((long long)n_pages * n_kv_heads * page_size < (1LL << 31),
                  "paged step: %d pages of %d rows x %d kv heads exceed 2^31 cache rows", n_pages, page_size,
                  n_kv_heads);
    ANELM_REQUIRE(max_seq_len > 0 && max_seq_len <= max_pages * page_size,
                  "paged step: max_seq_len %d beyond max_pages*page_size", max_seq_len);
    ANELM_REQUIRE(rot_dim >= 0 && rot_dim % 2 == 0 && rot_dim <= head_dim && rot_dim / 2 <= kMaxRotPairs,
                  "paged step: rot_dim %d must be even and <= head_dim", rot_dim);
    ANELM_REQUIRE(rope_mode == ANELM_ROPE_INTERLEAVED || rope_mode == ANELM_ROPE_HALF_SPLIT,
                  "paged step: rope_mode %d unknown", rope_mode);
    ANELM_REQUIRE(rope_table == nullptr || rope_rows > 0, "paged step: rope_rows %d", rope_rows);
    DecodeParams p{};
    p.out = out;
    p.q = q_gate;
    p.q_stride = 2 * head_dim;
    p.k_cache = k_pages;
    p.v_cache = v_pages;
    p.n_kv_heads = n_kv_heads;
    p.scale = 1.0f / sqrtf((float)head_dim);
    p.paged = 1;
    p.page_table = page_table;
    p.seq_lens = seq_lens;
    p.max_pages = max_pages;
    p.page_size = page_size;
    p.n_pages = n_pages;
    p.len = max_seq_len;
    p.fused = 1;
    p.q_norm_w = q_norm_w;
    p.k_norm_w = k_norm_w;
    p.k_new = k;
    p.v_new = v;
    p.k_cache_w = k_pages;
    p.v_cache_w = v_pages;
    p.eps = eps;
    p.rot_pairs = rot_dim / 2;
    p.rope_mode = rope_mode;
    p.gate = gate ? 1 : 0;
    p.positions = positions;
    p.rope_tab = rope_table;
    p.rope_rows = rope_table ? rope_rows : 0;
    p.theta = theta;
    return run_decode(p, ANELM_F16, n_heads, head_dim, n_seqs, max_seq_len, as_stream(stream));
}

extern "C" int anelm_rope_table(float* table, int rot_dim, int n_pos, float theta) {
    ANELM_NONNULL(table);
    ANELM_REQUIRE(rot_dim > 0 && rot_dim % 2 == 0 && rot_dim / 2 <= kMaxRotPairs, "rope_table: rot_dim %d", rot_dim);
    ANELM_REQUIRE(n_pos > 0, "rope_table: n_pos %d", n_pos);
    std::vector<float> host((size_t)n_pos * rot_dim);
    for (int pos = 0; pos < n_pos; pos++)
        rope_row(&host[(size_t)pos * rot_dim], &host[(size_t)pos * rot_dim + rot_dim / 2], rot_dim, pos, theta);
    ANELM_HIP(hipMemcpy(table, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice));
    return ANELM_OK;
}
