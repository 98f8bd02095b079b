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

// fp16 pair (lo, hi) and its dot product with another pair, accumulated in fp32
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_half2(float lo, float hi) {
    return (uint32_t)f2h(lo) | ((uint32_t)f2h(hi) << 16);
}
__device__ __forceinline__ float dot2_acc(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2v, a), __builtin_bit_cast(half2v, b), c, false);
}

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

// Paged decode over many sequences: a workgroup owns kPagedChunks chunks of
// 256/G keys of one (sequence, kv head) and walks them one after the other
// (online softmax across chunks: running maximum per head, rescaled sums).
// The split's page-table entries are read once into LDS.  Fewer, longer
// splits than the ring path also shrink the partial records 4x.
constexpr int kPagedChunks = 4;

template <typename KV, int D, int G>
__global__ __launch_bounds__(kNT) void attn_paged_kernel(const DecodeParams p) {
    constexpr int LPK = D / 8;        // lanes per key row (8 elements each)
    constexpr int KPI = 64 / LPK;     // key rows per wave instruction
    constexpr int KPB = kNW * KPI;    // key rows per workgroup instruction
    constexpr int KB = LPK / G;       // instructions per chunk
    constexpr int CK = KPB * KB;      // keys per chunk (= 256 / G)
    constexpr int KPS = CK * kPagedChunks;
    constexpr int REC = D + 2;
    static_assert(KB >= 1 && KB * G == LPK, "G must divide D/8");

    __shared__ __attribute__((aligned(16))) float sc_w[kNW][64];   // each wave's softmax weights of a chunk
    __shared__ float red_g[kNW][G];
    __shared__ float red_m[kNW][G];
    __shared__ float red_o[kNW][G][D];
    __shared__ int pg[KPS + 1];   // page-table entries of the split (any page size)
    // fused step only: q rows and the new key after norm + RoPE, RoPE row
    __shared__ float q_s[G][D];
    __shared__ float kn_s[D];
    __shared__ float red[kNW];
    __shared__ float rope_s[2][kMaxRotPairs];

    const int split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const int Hkv = p.n_kv_heads;
    const int tid = threadIdx.x;
    const int lane = tid & 63, w = tid >> 6;
    const int sub = lane / LPK, dl = lane % LPK;
    // fused: the sequence's new token is key `cached` and is attended too
    const int cached = p.seq_lens[seq];
    const int len = p.fused ? min(cached + 1, p.len) : min(cached, p.len);
    float* out = p.out + (size_t)seq * Hkv * G * D;
    if (len <= 0) {   // empty sequence: zeros, as cpu_ops.cpp:152-155
        if (split == 0)
            for (int e = tid; e < G * D; e += kNT) out[(size_t)kvh * G * D + e] = 0.f;
        return;
    }
    const int n_splits = (len + KPS - 1) / KPS;
    if (split >= n_splits) return;   // (uniform: before any barrier)
    const int k0 = split * KPS, nk_all = min(KPS, len - k0);
    const int nch = (nk_all + CK - 1) / CK;
    const float* q = p.q + (size_t)seq * Hkv * G * p.q_stride;

    const int ps = p.page_size;
    const int pfirst = k0 / ps, pcount = (k0 + nk_all - 1) / ps - pfirst + 1;
    const int32_t* ptab = p.page_table + (size_t)seq * p.max_pages;
    for (int i = tid; i < pcount; i += kNT) pg[i] = min(max(ptab[pfirst + i], 0), p.n_pages - 1);
    float qr[G][8];
    // fused: local index of the new key in this split (-1: another split's)
    const int t_new = p.fused && cached >= k0 && cached < k0 + nk_all ? cached - k0 : -1;
    if (p.fused) {
        // models/llm/qwen3_5.cpp:952-986 for this sequence: q/k RMSNorm, RoPE
        // at the token's position (the table row, or the same formula as
        // cpu_ops.cpp:51-55 past the table), fp16 append into the page
        const int pos = p.positions ? p.positions[seq] : cached;
        for (int j = tid; j < p.rot_pairs; j += kNT) {
            if (p.rope_tab != nullptr && pos >= 0 && pos < p.rope_rows) {
                rope_s[0][j] = p.rope_tab[(size_t)pos * 2 * p.rot_pairs + j];
                rope_s[1][j] = p.rope_tab[(size_t)pos * 2 * p.rot_pairs + p.rot_pairs + j];
            } else {
                const float freq = 1.0f / powf(p.theta, (float)(2 * j) / (float)(2 * p.rot_pairs));
                const float angle = (float)pos * freq;
                rope_s[0][j] = cosf(angle);
                rope_s[1][j] = sinf(angle);
            }
        }
        for (int e = tid; e < G * D; e += kNT) q_s[e / D][e % D] = q[(size_t)(kvh * G + e / D) * p.q_stride + e % D];
        __syncthreads();
        norm_rope_rows<D, G>(q_s, p.q_norm_w, p, red_g, rope_s[0], rope_s[1]);
        if (t_new >= 0) {
            const size_t nrow = ((size_t)seq * Hkv + kvh) * D;
            for (int d = tid; d < D; d += kNT) kn_s[d] = p.k_new[nrow + d];
            __syncthreads();
            norm_rope_row<D>(kn_s, p.k_norm_w, p, red, rope_s[0], rope_s[1]);
            const int page = pg[cached / ps - pfirst], row = cached % ps;
            const size_t off = (((size_t)page * Hkv + kvh) * ps + row) * D;
            KV* kw = reinterpret_cast<KV*>(p.k_cache_w) + off;
            KV* vw = reinterpret_cast<KV*>(p.v_cache_w) + off;
            for (int d = tid; d < D; d += kNT) {
                store_kv(kw + d, kn_s[d]);
                store_kv(vw + d, p.v_new[nrow + d]);
            }
        }
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) qr[g][i] = q_s[g][dl * 8 + i];
    } else {
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float* src = q + (size_t)(kvh * G + g) * p.q_stride + dl * 8;
#pragma unroll
            for (int i = 0; i < 8; i++) qr[g][i] = src[i];
        }
    }
    // fp16 caches: q as fp16 pairs, so scores are packed fp16 dot products
    // with fp32 accumulation (fp16 inputs, as the cache itself)
    constexpr bool kHalf = std::is_same<KV, uint16_t>::value;
    uint32_t qh[G][4];
    if constexpr (kHalf) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int j = 0; j < 4; j++) qh[g][j] = pack_half2(qr[g][2 * j], qr[g][2 * j + 1]);
    }
    lds_barrier();

    const KV* kc = reinterpret_cast<const KV*>(p.k_cache);
    const KV* vc = reinterpret_cast<const KV*>(p.v_cache);
    // rows past the split's last key load that key again (masked below): the
    // loads stay unconditional, so the counted waits stay exact.  A key's K
    // and V rows sit at the same offset of their caches.  The chunk's page
    // entries are all read from LDS before any address is formed (one wait),
    // a power-of-two page size takes shifts instead of divisions, and row
    // indices stay 32-bit (the host bounds the cache to 2^31 rows).
    const int ps_shift = (ps & (ps - 1)) == 0 ? __builtin_ctz((unsigned)ps) : -1;
    const unsigned rows_per_page = (unsigned)(Hkv * ps), head_row = (unsigned)(kvh * ps);
    auto load_rows = [&](int c, Raw8<KV> (&rk)[KB], Raw8<KV> (&rv)[KB]) __attribute__((always_inline)) {
        c = min(c, nch - 1);   // (past the last chunk: reload it, unused)
        unsigned kt[KB], page[KB], row[KB];
#pragma unroll
        for (int b = 0; b < KB; b++)   // key index inside the sequence
            kt[b] = (unsigned)(k0 + min(c * CK + b * KPB + w * KPI + sub, nk_all - 1));
        if (ps_shift >= 0) {
#pragma unroll
            for (int b = 0; b < KB; b++) {
                page[b] = (unsigned)pg[(int)(kt[b] >> ps_shift) - pfirst];
                row[b] = kt[b] & (unsigned)(ps - 1);
            }
        } else {
#pragma unroll
            for (int b = 0; b < KB; b++) {
                const unsigned pi = kt[b] / (unsigned)ps;
                page[b] = (unsigned)pg[(int)pi - pfirst];
                row[b] = kt[b] - pi * (unsigned)ps;
            }
        }
#pragma unroll
        for (int b = 0; b < KB; b++) {
            const size_t off = (size_t)(page[b] * rows_per_page + head_row + row[b]) * D + dl * 8;
            rk[b] = load_raw(kc + off);
            rv[b] = load_raw(vc + off);
        }
    };

    // Online softmax per wave: a wave keeps its own running maximum per head
    // and sums over the keys it holds (rows t = b*KPB + w*KPI + sub of each
    // chunk), so the chunk loop has no workgroup barrier and a wave waiting
    // on its rows holds up no other; the waves' states are merged once at the
    // end by log-sum-exp.  After the transpose reduction lane (sub, dl) holds
    // the score of row b = dl / G for head g = dl % G = lane % G.
    float m[G], acc[G][8];
    float lsum = 0.f;   // this lane's share of the sum for its head lane % G
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
#pragma unroll
        for (int i = 0; i < 8; i++) acc[g][i] = 0.f;
    }
    float* pw = sc_w[w];
    const int g_own = dl % G;
    auto chunk = [&](int c, const Raw8<KV> (&rk)[KB], const Raw8<KV> (&rv)[KB]) __attribute__((always_inline)) {
        const int nk = min(CK, nk_all - c * CK);
        // ---- scores: one transpose reduction over the KB rows of each lane
        float s_own;
        {
            float part[KB * G];
#pragma unroll
            for (int b = 0; b < KB; b++) {
                if constexpr (kHalf) {
                    const uint32_t kw[4] = {rk[b].a.x, rk[b].a.y, rk[b].a.z, rk[b].a.w};
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        float sv = 0.f;
#pragma unroll
                        for (int j = 0; j < 4; j++) sv = dot2_acc(qh[g][j], kw[j], sv);
                        part[b * G + g] = sv;
                    }
                } else {
                    float kf[8];
                    to_f32(rk[b], kf);
#pragma unroll
                    for (int g = 0; g < G; g++) {
                        float sv = 0.f;
#pragma unroll
                        for (int i = 0; i < 8; i++) sv = fmaf(qr[g][i], kf[i], sv);
                        part[b * G + g] = sv;
                    }
                }
            }
            transpose_reduce<LPK, KB * G>(part, dl);
            const int t = (dl / G) * KPB + w * KPI + sub;
            s_own = t < nk ? part[0] * p.scale : -INFINITY;
        }
        // ---- running maximum per head over the wave's keys (exact XOR
        // partners keep the lanes of one head together)
        float mx = s_own;
#pragma unroll
        for (int mm = G; mm < 64; mm <<= 1) mx = fmaxf(mx, shfl_xor(mx, mm));
        float alpha_own = 0.f, m_own = 0.f;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const float mc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mx), g));
            const float m_new = fmaxf(m[g], mc);
            const float m_use = m_new == -INFINITY ? 0.f : m_new;   // no valid key yet: weights 0
            const float alpha = __expf(m[g] - m_use);              // 0 while m is -inf
#pragma unroll
            for (int i = 0; i < 8; i++) acc[g][i] *= alpha;
            m[g] = m_new;
            if (g == g_own) {
                alpha_own = alpha;
                m_own = m_use;
            }
        }
        const float e = __expf(s_own - m_own);   // masked keys: exp(-inf) = 0
        lsum = lsum * alpha_own + e;
        // the weights back in row order through the wave's own LDS (a wave's
        // LDS accesses execute in order: no barrier)
        pw[lane] = e;
        float pv[KB * G];
#pragma unroll
        for (int k = 0; k < KB * G / 4; k++) {
            const float4 v4 = *reinterpret_cast<const float4*>(pw + sub * LPK + 4 * k);
            pv[4 * k] = v4.x;
            pv[4 * k + 1] = v4.y;
            pv[4 * k + 2] = v4.z;
            pv[4 * k + 3] = v4.w;
        }
        // ---- P V (fp16 caches: two key rows per packed dot product, the
        // weights rounded to fp16 pairs and the rows' values interleaved)
        constexpr int KP = kHalf ? KB / 2 : 0;
        if constexpr (kHalf) {
#pragma unroll
            for (int j = 0; j < KP; j++) {
                const uint32_t va[4] = {rv[2 * j].a.x, rv[2 * j].a.y, rv[2 * j].a.z, rv[2 * j].a.w};
                const uint32_t vb[4] = {rv[2 * j + 1].a.x, rv[2 * j + 1].a.y, rv[2 * j + 1].a.z,
                                        rv[2 * j + 1].a.w};
                uint32_t vp[8];   // (row 2j, row 2j+1) of dims 2k and 2k+1
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    vp[2 * k] = __builtin_amdgcn_perm(vb[k], va[k], 0x05040100u);
                    vp[2 * k + 1] = __builtin_amdgcn_perm(vb[k], va[k], 0x07060302u);
                }
#pragma unroll
                for (int g = 0; g < G; g++) {
                    const uint32_t pp = pack_half2(pv[(2 * j) * G + g], pv[(2 * j + 1) * G + g]);
#pragma unroll
                    for (int i = 0; i < 8; i++) acc[g][i] = dot2_acc(pp, vp[i], acc[g][i]);
                }
            }
        }
#pragma unroll
        for (int b = 2 * KP; b < KB; b++) {
            float vf[8];
            to_f32(rv[b], vf);
#pragma unroll
            for (int g = 0; g < G; g++) {
                const float pgv = pv[b * G + g];
#pragma unroll
                for (int i = 0; i < 8; i++) acc[g][i] = fmaf(pgv, vf[i], acc[g][i]);
            }
        }
    };

    // one chunk's rows in registers at a time (several workgroups per CU hide
    // each other's load latency)
    for (int c = 0; c < nch; c++) {
        Raw8<KV> rk[KB], rv[KB];
        load_rows(c, rk, rv);
        if (t_new >= 0 && c == t_new / CK) {
            // the new key's row was loaded before (or while) it was stored:
            // take it from the prologue, rounded as stored
#pragma unroll
            for (int b = 0; b < KB; b++) {
                if (c * CK + b * KPB + w * KPI + sub == t_new) {
                    rk[b] = make_raw<KV>(kn_s + dl * 8);
                    rv[b] = make_raw<KV>(p.v_new + ((size_t)seq * Hkv + kvh) * D + dl * 8);
                }
            }
        }
        chunk(c, rk, rv);
    }

    // ---- merge the waves: per head M = max of the waves' maxima, each wave
    // weighed by e^(m_w - M); O summed over the lanes sharing dims first
    float lw[G];
    {
        float l = lsum;
#pragma unroll
        for (int mm = G; mm < 64; mm <<= 1) l += shfl_xor(l, mm);
#pragma unroll
        for (int g = 0; g < G; g++) lw[g] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(l), g));
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) {
            red_g[w][g] = lw[g];
            red_m[w][g] = m[g];
        }
    }
#pragma unroll
    for (int mm = LPK; mm < 64; mm <<= 1)
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) acc[g][i] += shfl_xor(acc[g][i], mm);
    if (sub == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int i = 0; i < 8; i++) red_o[w][g][dl * 8 + i] = acc[g][i];
    }
    lds_barrier();
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
    if (n_splits == 1) {
        for (int e = tid; e < G * D; e += kNT) {
            const int g = e / D, d = e % D;
            float o = 0.f;
#pragma unroll
            for (int ww = 0; ww < kNW; ww++) o += red_o[ww][g][d] * wsc[g][ww];
            const int hq = kvh * G + g;
            float yv = o / ltot[g];
            if (p.gate) yv = yv / (1.0f + expf(-q[(size_t)hq * p.q_stride + D + d]));
            out[(size_t)hq * D + d] = yv;
        }
        return;
    }
    float* rec = p.part + (((size_t)seq * Hkv + kvh) * p.max_splits + split) * G * REC;
    for (int e = tid; e < G * D; e += kNT) {
        const int g = e / D, d = e % D;
        float o = 0.f;
#pragma unroll
        for (int ww = 0; ww < kNW; ww++) o += red_o[ww][g][d] * wsc[g][ww];
        rec[(size_t)g * REC + 2 + d] = o;
        if (d == 0) { rec[(size_t)g * REC] = mtot[g]; rec[(size_t)g * REC + 1] = ltot[g]; }
    }
}

// Log-sum-exp merge of the split partials of one (sequence, q head) for 64
// output dims per workgroup: M = max m_s, L = sum l_s e^(m_s-M),
// O = sum o_s e^(m_s-M), out = O / L, then the sigmoid gate.  The 256
// threads first turn all m_s into weights e^(m_s-M) in LDS, then four groups
// of 64 threads sum interleaved quarters of the splits.
constexpr int kCombineChunk = 1024;   // splits weighed per LDS pass

template <int D, int G>
__global__ __launch_bounds__(256) void attn_combine_kernel(const DecodeParams p) {
    constexpr int REC = D + 2;
    __shared__ float f[kCombineChunk];
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
    float M = -INFINITY;
    for (int s = tid; s < n; s += 256) M = fmaxf(M, base[(size_t)s * rs]);
    M = block_max<256>(M, red);
    float L = 0.f, O = 0.f;
    for (int c0 = 0; c0 < n; c0 += kCombineChunk) {
        const int cn = min(kCombineChunk, n - c0);
        float lpart = 0.f;
        for (int s = tid; s < cn; s += 256) {
            const float* r = base + (size_t)(c0 + s) * rs;
            const float w = __expf(r[0] - M);
            f[s] = w;
            lpart += r[1] * w;
        }
        L += block_sum<256>(lpart, red);   // (its barriers also publish f)
        int s = grp;
        for (; s + 12 < cn; s += 16) {
            const float o0 = base[(size_t)(c0 + s) * rs + 2 + d];
            const float o1 = base[(size_t)(c0 + s + 4) * rs + 2 + d];
            const float o2 = base[(size_t)(c0 + s + 8) * rs + 2 + d];
            const float o3 = base[(size_t)(c0 + s + 12) * rs + 2 + d];
            O += f[s] * o0 + f[s + 4] * o1 + f[s + 8] * o2 + f[s + 12] * o3;
        }
        for (; s < cn; s += 4) O += f[s] * base[(size_t)(c0 + s) * rs + 2 + d];
        __syncthreads();
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
        hipLaunchKernelGGL((attn_paged_kernel<KV, D, G>), grid, dim3(kNT), 0, st, p);
        ANELM_LAUNCHED("attn_paged_kernel");
    } else {
        hipLaunchKernelGGL((attn_decode_kernel<KV, D, G>), grid, dim3(ring_threads<G>()), 0, st, p);
        ANELM_LAUNCHED("attn_decode_kernel");
    }
    if (p.max_splits > 1 && p.arrivals == nullptr) {
        dim3 cgrid(D / 64, grid.y * G, grid.z);
        hipLaunchKernelGGL((attn_combine_kernel<D, G>), cgrid, dim3(256), 0, st, p);
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
    const int kps = (256 / G) * (paged ? kPagedChunks : 1);
    const int max_splits = (max_len + kps - 1) / kps;
    if (max_splits <= 1) return 0;
    return (size_t)n_seqs * n_kv_heads * max_splits * G * (D + 2) * sizeof(float);
}

// Sets the split layout and partials buffer for one decode call, then
// launches.  A split is 256/G keys (ring mode: every lane of the workgroup
// then loads all of its K and V rows at once) or kPagedChunks such chunks
// (paged mode).  `max_len` bounds every sequence's key count; `n_seqs`
// sequences (1 in ring mode).  The partials go to `part` (part_cap bytes)
// when it is given, else to the library workspace.
int run_decode(DecodeParams& p, int kv_dtype, int n_heads, int D, int n_seqs, int max_len,
               hipStream_t st, float* part = nullptr, size_t part_cap = 0) {
    const int Hkv = p.n_kv_heads;
    const int G = n_heads / Hkv;
    const int kps = (256 / G) * (p.paged ? kPagedChunks : 1);
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
    if (need > 0 && part != nullptr) {
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
