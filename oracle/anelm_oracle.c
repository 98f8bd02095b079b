/*
 * anelm_oracle.c -- CPU restatement of ANE-LM's core/cpu_ops hot path.
 *
 * TEST INFRASTRUCTURE ONLY (the oracle).  Loaded by tests/, smoke() and the
 * cpu_baseline leg of bench.py; never by the product library.
 *
 * Accelerate calls in the reference are restated from their documented
 * definitions as sequential fp32 loops:
 *   vDSP_svesq  -> s = sum x[i]^2          vDSP_vsmul -> out[i] = x[i]*s
 *   vDSP_vmul   -> out[i] = a[i]*b[i]      vDSP_dotpr -> s = sum a[i]*b[i]
 *   vDSP_vneg/vvexpf/vDSP_vsadd/vDSP_vdiv  -> y[i] = y[i] / (1 + expf(-z[i]))
 *   cblas_sgemv  -> y[i] = sum_j A[i][j] x[j]  (NoTrans) / sum_i A[i][j] x[i] (Trans)
 *   cblas_sscal / cblas_sger / cblas_saxpy -> elementwise definitions.
 * Build flags keep IEEE semantics (no -ffast-math, -ffp-contract=off).
 */
#include "anelm_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ fp16 */

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                       /* subnormal: m * 2^-24, renormalise */
            int ee = 113;              /* exponent field of 2^-14 */
            while (!(m & 0x400u)) { m <<= 1; ee--; }
            m &= 0x3ffu;
            bits = sign | ((uint32_t)ee << 23) | (m << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu)); /* NaN */
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 -> inf */
    uint32_t e = ax >> 23;
    if (e < 113) {                      /* result is subnormal or zero */
        if (e < 102) return sign;       /* < 2^-25 rounds to zero */
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;      /* value / 2^-24 = m >> shift */
        uint32_t r = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (r & 1u))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((e - 112u) << 10) | ((ax >> 13) & 0x3ffu);
    uint32_t rem = ax & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) r++;
    return (uint16_t)(sign | r);
}

void orc_f16_to_f32_array(float* out, const uint16_t* in, long n) {
    for (long i = 0; i < n; i++) out[i] = orc_f16_to_f32(in[i]);
}

void orc_f32_to_f16_array(uint16_t* out, const float* in, long n) {
    for (long i = 0; i < n; i++) out[i] = orc_f32_to_f16(in[i]);
}

/* ------------------------------------------------------------- cpu_ops */

/* core/cpu_ops.cpp:6-13: x = x / (1 + exp(-x)) */
void orc_silu_vec_inplace(float* x, int n) {
    for (int i = 0; i < n; i++) {
        float t = expf(-x[i]) + 1.0f;
        x[i] = x[i] / t;
    }
}

/* core/cpu_ops.cpp:15-22: y = y / (1 + exp(-z)) */
void orc_mul_sigmoid_inplace(float* y, const float* z, int n) {
    for (int i = 0; i < n; i++) {
        float t = expf(-z[i]) + 1.0f;
        y[i] = y[i] / t;
    }
}

/* core/cpu_ops.cpp:24-30 */
void orc_rmsnorm(float* out, const float* x, const float* w, int dim, float eps) {
    float ss = 0.0f;
    for (int i = 0; i < dim; i++) ss += x[i] * x[i];
    ss = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; i++) out[i] = x[i] * ss;
    for (int i = 0; i < dim; i++) out[i] = out[i] * w[i];
}

/* core/cpu_ops.cpp:32-38: rmsnorm (default eps 1e-6), then * sigmoid(z), then * z */
void orc_rmsnorm_gated(float* out, const float* x, const float* z, const float* w, int dim) {
    orc_rmsnorm(out, x, w, dim, 1e-6f);
    orc_mul_sigmoid_inplace(out, z, dim);
    for (int i = 0; i < dim; i++) out[i] = out[i] * z[i];
}

/* core/cpu_ops.cpp:40-63 (interleaved pairs); half-split variant follows
 * scripts/serve_hybrid.py:94-103.  cos/sin for pair j at dim i = 2j:
 * cosf(pos * (1 / powf(theta, i / rot_dim))), identical to the table built at
 * models/llm/qwen3_5.cpp:308-324. */
void orc_apply_rope(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                    int q_head_stride, int k_head_stride, int rot_dim, int pos, float theta,
                    const float* cos_row, const float* sin_row, int rope_mode) {
    (void)head_dim;
    int half = rot_dim / 2;
    for (int h = 0; h < n_q_heads + n_kv_heads; h++) {
        float* v = (h < n_q_heads) ? q + (long)h * q_head_stride
                                   : k + (long)(h - n_q_heads) * k_head_stride;
        for (int i = 0, j = 0; i < rot_dim; i += 2, j++) {
            float cos_a, sin_a;
            if (cos_row && sin_row) {
                cos_a = cos_row[j];
                sin_a = sin_row[j];
            } else {
                float freq = 1.0f / powf(theta, (float)i / (float)rot_dim);
                float angle = (float)pos * freq;
                cos_a = cosf(angle);
                sin_a = sinf(angle);
            }
            int i0 = (rope_mode == 0) ? i : j;
            int i1 = (rope_mode == 0) ? i + 1 : j + half;
            float v0 = v[i0];
            float v1 = v[i1];
            v[i0] = v0 * cos_a - v1 * sin_a;
            v[i1] = v0 * sin_a + v1 * cos_a;
        }
    }
}

/* models/llm/qwen3_5.cpp:308-324 */
void orc_rope_table(float* cos_tab, float* sin_tab, int max_pos, int rot_dim, float theta) {
    int half = rot_dim / 2;
    float* inv_freq = (float*)malloc(sizeof(float) * (size_t)half);
    for (int j = 0, i = 0; i < rot_dim; i += 2, j++)
        inv_freq[j] = 1.0f / powf(theta, (float)i / (float)rot_dim);
    for (int p = 0; p < max_pos; p++)
        for (int j = 0; j < half; j++) {
            float angle = (float)p * inv_freq[j];
            cos_tab[(long)p * half + j] = cosf(angle);
            sin_tab[(long)p * half + j] = sinf(angle);
        }
    free(inv_freq);
}

/* core/cpu_ops.cpp:65-75 */
void orc_softmax(float* x, int n) {
    float max_val = x[0];
    for (int i = 1; i < n; i++) if (x[i] > max_val) max_val = x[i];
    float sum = 0.0f;
    for (int i = 0; i < n; i++) {
        x[i] = expf(x[i] - max_val);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] = x[i] * inv;
}

/* core/cpu_ops.cpp:77-80: row-major sgemv NoTrans */
void orc_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim) {
    for (int r = 0; r < out_dim; r++) {
        const float* row = W + (long)r * in_dim;
        float s = 0.0f;
        for (int c = 0; c < in_dim; c++) s += row[c] * x[c];
        y[r] = s;
    }
}

/* core/cpu_ops.cpp:82-87: x *= 1 / sqrtf(sum x^2 + 1e-12) */
void orc_l2_normalize(float* x, int dim) {
    float norm = 0.0f;
    for (int i = 0; i < dim; i++) norm += x[i] * x[i];
    norm = 1.0f / sqrtf(norm + 1e-12f);
    for (int i = 0; i < dim; i++) x[i] = x[i] * norm;
}

/* core/cpu_ops.cpp:89-129: depthwise causal conv over a ring of kernel-1
 * past inputs per channel; state layout [channels][kernel-1], ring head
 * *state_pos.  The kernel_size == 4 fast path (:94-110) and the generic path
 * (:111-124) compute the same sum; both are restated by the generic loop. */
void orc_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                       const float* w, int channels, int kernel_size) {
    int state_len = kernel_size - 1;
    int pos = *state_pos;
    for (int c = 0; c < channels; c++) {
        float sum = 0.0f;
        int base = c * state_len;
        for (int j = 0; j < state_len; j++) {
            int idx = pos + j;
            if (idx >= state_len) idx -= state_len;
            sum += conv_state[base + idx] * w[c * kernel_size + j];
        }
        float xc = x[c];
        y[c] = sum + xc * w[c * kernel_size + state_len];
        conv_state[base + pos] = xc;
    }
    pos++;
    if (pos == state_len) pos = 0;
    *state_pos = pos;
}

/* core/cpu_ops.cpp:131-146 (order 0):
 *   Sk = S^T k ; delta = v - Sk ; S = decay*S ; S += beta * k delta^T ; y = S^T q
 * order 1 = transformers recurrent rule (scripts/export_hybrid_chunks.py:137-147):
 *   S = decay*S ; delta = beta*(v - S^T k) ; S += k delta^T ; y = S^T q        */
void orc_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                  float decay, float beta, int key_dim, int value_dim, int order) {
    float* Sk = (float*)malloc(sizeof(float) * (size_t)value_dim);
    float* delta = (float*)malloc(sizeof(float) * (size_t)value_dim);
    long n = (long)key_dim * value_dim;
    if (order == 0) {
        for (int j = 0; j < value_dim; j++) Sk[j] = 0.0f;
        for (int i = 0; i < key_dim; i++)
            for (int j = 0; j < value_dim; j++) Sk[j] += state[(long)i * value_dim + j] * k[i];
        for (int j = 0; j < value_dim; j++) delta[j] = v[j] - Sk[j];
        for (long e = 0; e < n; e++) state[e] = decay * state[e];
        for (int i = 0; i < key_dim; i++) {
            float bk = beta * k[i];
            for (int j = 0; j < value_dim; j++) state[(long)i * value_dim + j] += bk * delta[j];
        }
    } else {
        for (long e = 0; e < n; e++) state[e] = decay * state[e];
        for (int j = 0; j < value_dim; j++) Sk[j] = 0.0f;
        for (int i = 0; i < key_dim; i++)
            for (int j = 0; j < value_dim; j++) Sk[j] += state[(long)i * value_dim + j] * k[i];
        for (int j = 0; j < value_dim; j++) delta[j] = (v[j] - Sk[j]) * beta;
        for (int i = 0; i < key_dim; i++)
            for (int j = 0; j < value_dim; j++) state[(long)i * value_dim + j] += k[i] * delta[j];
    }
    for (int j = 0; j < value_dim; j++) y[j] = 0.0f;
    for (int i = 0; i < key_dim; i++)
        for (int j = 0; j < value_dim; j++) y[j] += state[(long)i * value_dim + j] * q[i];
    free(Sk);
    free(delta);
}

/* core/cpu_ops.cpp:148-204 */
void orc_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                       int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                       int cache_start, int cache_len, int cache_capacity) {
    if (cache_len <= 0) {
        memset(out, 0, (size_t)n_heads * head_dim * sizeof(float));
        return;
    }
    int groups = n_heads / n_kv_heads;
    float scale = 1.0f / sqrtf((float)head_dim);
    long kv_step = (long)n_kv_heads * head_dim;
    int first_span = cache_capacity - cache_start;
    if (first_span > cache_len) first_span = cache_len;
    int second_span = cache_len - first_span;
    float* scores = (float*)malloc((size_t)cache_len * sizeof(float));
    for (int h = 0; h < n_heads; h++) {
        int kv_h = h / groups;
        const float* qh = q + (long)h * q_head_stride;
        float* oh = out + (long)h * head_dim;
        long off = (long)kv_h * head_dim;
        int t = 0;
        for (int s = 0; s < first_span; s++, t++) {
            const float* kh = k_cache + (long)(cache_start + s) * kv_step + off;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; d++) dot += qh[d] * kh[d];
            scores[t] = dot * scale;
        }
        for (int s = 0; s < second_span; s++, t++) {
            const float* kh = k_cache + (long)s * kv_step + off;
            float dot = 0.0f;
            for (int d = 0; d < head_dim; d++) dot += qh[d] * kh[d];
            scores[t] = dot * scale;
        }
        orc_softmax(scores, cache_len);
        for (int d = 0; d < head_dim; d++) oh[d] = 0.0f;
        t = 0;
        for (int s = 0; s < first_span; s++, t++) {
            const float* vh = v_cache + (long)(cache_start + s) * kv_step + off;
            float sv = scores[t];
            for (int d = 0; d < head_dim; d++) oh[d] += sv * vh[d];
        }
        for (int s = 0; s < second_span; s++, t++) {
            const float* vh = v_cache + (long)s * kv_step + off;
            float sv = scores[t];
            for (int d = 0; d < head_dim; d++) oh[d] += sv * vh[d];
        }
    }
    free(scores);
}

/* --------------------------------------------------------- compositions */

/* models/llm/qwen3_5.cpp:944-1002 with the cache stored as fp16: q/k RMSNorm
 * per head (:952-959), RoPE (:961-971), ring append (:973-986), gqa_attention
 * (:989-991), sigmoid output gate (:993-1000).  The cache is widened exactly to
 * fp32 before attention, so the arithmetic is the reference's on the fp16
 * values. */
void orc_full_attn_decode(float* out, float* q_gate, float* k, const float* v,
                          uint16_t* k_cache, uint16_t* v_cache,
                          const float* q_norm_w, const float* k_norm_w,
                          int n_heads, int n_kv_heads, int head_dim, int rot_dim,
                          int pos, float theta, float eps, int rope_mode, int gate,
                          int* cache_start, int* cache_len, int cache_capacity) {
    int D = head_dim;
    /* NULL norm weights: q and k arrive normalised (scripts/serve_hybrid.py:89-107
     * applies RoPE only) */
    if (q_norm_w) {
        for (int h = 0; h < n_heads; h++) {
            float* qh = q_gate + (long)h * 2 * D;
            orc_rmsnorm(qh, qh, q_norm_w, D, eps);
        }
    }
    if (k_norm_w)
        for (int h = 0; h < n_kv_heads; h++) orc_rmsnorm(k + (long)h * D, k + (long)h * D, k_norm_w, D, eps);
    orc_apply_rope(q_gate, k, n_heads, n_kv_heads, D, 2 * D, D, rot_dim, pos, theta, 0, 0, rope_mode);

    int slot;
    if (*cache_len < cache_capacity) {
        slot = *cache_start + *cache_len;
        if (slot >= cache_capacity) slot -= cache_capacity;
        (*cache_len)++;
    } else {
        slot = *cache_start;
        (*cache_start)++;
        if (*cache_start >= cache_capacity) *cache_start = 0;
    }
    long kv_stride = (long)n_kv_heads * D;
    orc_f32_to_f16_array(k_cache + (long)slot * kv_stride, k, kv_stride);
    orc_f32_to_f16_array(v_cache + (long)slot * kv_stride, v, kv_stride);

    long total = (long)cache_capacity * kv_stride;
    float* kf = (float*)malloc(sizeof(float) * (size_t)total);
    float* vf = (float*)malloc(sizeof(float) * (size_t)total);
    orc_f16_to_f32_array(kf, k_cache, total);
    orc_f16_to_f32_array(vf, v_cache, total);
    orc_gqa_attention(out, q_gate, kf, vf, n_heads, n_kv_heads, D, 2 * D,
                      *cache_start, *cache_len, cache_capacity);
    free(kf);
    free(vf);
    if (gate) {
        for (int h = 0; h < n_heads; h++)
            orc_mul_sigmoid_inplace(out + (long)h * D, q_gate + (long)h * 2 * D + D, D);
    }
}

/* models/llm/qwen3_5.cpp:879-908: per key head l2-normalise q and k and scale
 * q by 1/sqrt(dk) (:882-887); per value head beta = sigmoid(b),
 * decay = exp(-A * softplus(a + dt_bias)) (:896-898, cpu_ops.h:13-14), key head
 * h / (Hv/Hk) (:890), ssm_step (:899); optional rmsnorm_gated (:902-908). */
void orc_deltanet_decode(float* y, float* state, float* q, float* k, const float* v,
                         const float* a, const float* b, const float* A, const float* dt_bias,
                         const float* z, const float* norm_w,
                         int Hk, int Hv, int dk, int dv, int flags) {
    float q_scale = 1.0f / sqrtf((float)dk);
    int group = Hv / Hk;
    if (flags & 1) {
        for (int kh = 0; kh < Hk; kh++) {
            orc_l2_normalize(q + (long)kh * dk, dk);
            orc_l2_normalize(k + (long)kh * dk, dk);
            for (int i = 0; i < dk; i++) q[(long)kh * dk + i] = q[(long)kh * dk + i] * q_scale;
        }
    } else {
        for (int kh = 0; kh < Hk; kh++)
            for (int i = 0; i < dk; i++) q[(long)kh * dk + i] = q[(long)kh * dk + i] * q_scale;
    }
    float* ytmp = (float*)malloc(sizeof(float) * (size_t)dv);
    for (int h = 0; h < Hv; h++) {
        int kh = (group > 1) ? h / group : h;
        float beta = 1.0f / (1.0f + expf(-b[h]));
        float sp = logf(1.0f + expf(a[h] + dt_bias[h]));
        float decay = expf(-A[h] * sp);
        orc_ssm_step(ytmp, state + (long)h * dk * dv, q + (long)kh * dk, k + (long)kh * dk,
                     v + (long)h * dv, decay, beta, dk, dv, (flags & 2) ? 1 : 0);
        if (flags & 4) {
            orc_rmsnorm_gated(y + (long)h * dv, ytmp, z + (long)h * dv, norm_w, dv);
        } else {
            memcpy(y + (long)h * dv, ytmp, sizeof(float) * (size_t)dv);
        }
    }
    free(ytmp);
}

/* generate.cpp:76-84 / qwen3_5.cpp:1204-1217: prefill runs the decode core per
 * token, so row t is gqa_attention over keys 0..t (cache_len = t+1). */
void orc_prefill_attention(float* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           int S, int Hq, int Hkv, int D, int row_begin, int row_end) {
    long kvn = (long)S * Hkv * D;
    float* kf = (float*)malloc(sizeof(float) * (size_t)kvn);
    float* vf = (float*)malloc(sizeof(float) * (size_t)kvn);
    float* qf = (float*)malloc(sizeof(float) * (size_t)Hq * D);
    orc_f16_to_f32_array(kf, k, kvn);
    orc_f16_to_f32_array(vf, v, kvn);
    for (int t = row_begin; t < row_end; t++) {
        orc_f16_to_f32_array(qf, q + (long)t * Hq * D, (long)Hq * D);
        orc_gqa_attention(out + (long)(t - row_begin) * Hq * D, qf, kf, vf, Hq, Hkv, D, D, 0, t + 1, S);
    }
    free(kf);
    free(vf);
    free(qf);
}

/* T sequential DeltaNet decode steps (qwen3_5.cpp:1204-1217 runs the core per
 * token during prefill). */
void orc_deltanet_prefill(float* y, float* state, float* q, float* k, const float* v,
                          const float* a, const float* b, const float* A, const float* dt_bias,
                          int S, int Hk, int Hv, int dk, int dv, int flags) {
    for (int t = 0; t < S; t++) {
        orc_deltanet_decode(y + (long)t * Hv * dv, state, q + (long)t * Hk * dk, k + (long)t * Hk * dk,
                            v + (long)t * Hv * dv, a + (long)t * Hv, b + (long)t * Hv, A, dt_bias,
                            0, 0, Hk, Hv, dk, dv, flags & 3);
    }
}

/* --------------------------------------------------------------- LUT6 */
/* Index k of a row occupies bits [6k, 6k+6) of the little-endian byte stream:
 * 4 indices per 3 bytes, LSB first (the sub-byte order of the reference's LUT4
 * packing, core/ane_runtime.cpp:1047-1048, extended to 6 bits). */

void orc_lut6_pack(uint8_t* packed, const uint8_t* idx, long n) {
    for (long g = 0; g < n / 4; g++) {
        uint32_t i0 = idx[4 * g] & 63u, i1 = idx[4 * g + 1] & 63u;
        uint32_t i2 = idx[4 * g + 2] & 63u, i3 = idx[4 * g + 3] & 63u;
        uint32_t w = i0 | (i1 << 6) | (i2 << 12) | (i3 << 18);
        packed[3 * g] = (uint8_t)(w & 0xffu);
        packed[3 * g + 1] = (uint8_t)((w >> 8) & 0xffu);
        packed[3 * g + 2] = (uint8_t)((w >> 16) & 0xffu);
    }
}

void orc_lut6_unpack(uint8_t* idx, const uint8_t* packed, long n) {
    for (long g = 0; g < n / 4; g++) {
        uint32_t b0 = packed[3 * g], b1 = packed[3 * g + 1], b2 = packed[3 * g + 2];
        idx[4 * g] = (uint8_t)(b0 & 63u);
        idx[4 * g + 1] = (uint8_t)((b0 >> 6) | ((b1 & 15u) << 2));
        idx[4 * g + 2] = (uint8_t)((b1 >> 4) | ((b2 & 3u) << 4));
        idx[4 * g + 3] = (uint8_t)(b2 >> 2);
    }
}

void orc_lut6_dequant_row(float* w, const uint8_t* packed_row, const uint16_t* lut64, int in_dim) {
    for (int g = 0; g < in_dim / 4; g++) {
        uint32_t b0 = packed_row[3 * g], b1 = packed_row[3 * g + 1], b2 = packed_row[3 * g + 2];
        w[4 * g] = orc_f16_to_f32(lut64[b0 & 63u]);
        w[4 * g + 1] = orc_f16_to_f32(lut64[(b0 >> 6) | ((b1 & 15u) << 2)]);
        w[4 * g + 2] = orc_f16_to_f32(lut64[(b1 >> 4) | ((b2 & 3u) << 4)]);
        w[4 * g + 3] = orc_f16_to_f32(lut64[b2 >> 2]);
    }
}

/* matvec (core/cpu_ops.cpp:77-80) on the dequantised rows; row r uses the
 * 64-entry fp16 LUT of its 32-row group r/32.  The input vector is rounded to
 * fp16 first (round to nearest even): the reference runs its LUT6 matrices
 * only inside CoreML models whose inputs are fp16 (scripts/export_hybrid_chunks.py:507
 * declares x float16; core/coreml_runtime.cpp:331-336 converts the fp32
 * activations with vImageConvert_PlanarFtoPlanar16F).  Products and the sum
 * are fp32. */
void orc_lut6_matvec(float* y, const uint8_t* packed, const uint16_t* lut, const float* x,
                     int out_dim, int in_dim, int row_begin, int row_end) {
    (void)out_dim;
    float* w = (float*)malloc(sizeof(float) * (size_t)in_dim);
    float* xh = (float*)malloc(sizeof(float) * (size_t)in_dim);
    for (int c = 0; c < in_dim; c++) xh[c] = orc_f16_to_f32(orc_f32_to_f16(x[c]));
    long row_bytes = (long)in_dim * 3 / 4;
    for (int r = row_begin; r < row_end; r++) {
        orc_lut6_dequant_row(w, packed + (long)r * row_bytes, lut + (long)(r / 32) * 64, in_dim);
        float s = 0.0f;
        for (int c = 0; c < in_dim; c++) s += w[c] * xh[c];
        y[r - row_begin] = s;
    }
    free(xh);
    free(w);
}

/* orc_lut6_matvec for `batch` inputs x [batch][in_dim] -> y [batch][out_dim]:
 * each row is dequantised once and every input's sum runs over the columns
 * in the same order as orc_lut6_matvec (the loop over the inputs is the
 * inner one), so y[b] equals orc_lut6_matvec of x[b] bit for bit. */
void orc_lut6_matvec_batch(float* y, const uint8_t* packed, const uint16_t* lut, const float* x,
                           int batch, int out_dim, int in_dim) {
    float* w = (float*)malloc(sizeof(float) * (size_t)in_dim);
    float* xt = (float*)malloc(sizeof(float) * (size_t)in_dim * batch);
    float* acc = (float*)malloc(sizeof(float) * (size_t)batch);
    for (int b = 0; b < batch; b++)
        for (int c = 0; c < in_dim; c++)
            xt[(size_t)c * batch + b] = orc_f16_to_f32(orc_f32_to_f16(x[(size_t)b * in_dim + c]));
    long row_bytes = (long)in_dim * 3 / 4;
    for (int r = 0; r < out_dim; r++) {
        orc_lut6_dequant_row(w, packed + (long)r * row_bytes, lut + (long)(r / 32) * 64, in_dim);
        for (int b = 0; b < batch; b++) acc[b] = 0.0f;
        for (int c = 0; c < in_dim; c++) {
            const float wc = w[c];
            const float* xc = xt + (size_t)c * batch;
            for (int b = 0; b < batch; b++) acc[b] += wc * xc[b];
        }
        for (int b = 0; b < batch; b++) y[(size_t)b * out_dim + r] = acc[b];
    }
    free(acc);
    free(xt);
    free(w);
}

/* SwiGLU FFN (models/llm/qwen3_5.cpp:1118-1130): down(silu(gate x) * (up x)).
 * scratch holds 2*inter floats. */
void orc_lut6_ffn(float* y, const uint8_t* gate_w, const uint16_t* gate_lut,
                  const uint8_t* up_w, const uint16_t* up_lut,
                  const uint8_t* down_w, const uint16_t* down_lut,
                  const float* x, int hidden, int inter, float* scratch) {
    float* g = scratch;
    float* u = scratch + inter;
    orc_lut6_matvec(g, gate_w, gate_lut, x, inter, hidden, 0, inter);
    orc_lut6_matvec(u, up_w, up_lut, x, inter, hidden, 0, inter);
    for (int i = 0; i < inter; i++) {
        float gv = g[i];
        g[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
    orc_lut6_matvec(y, down_w, down_lut, g, hidden, inter, 0, hidden);
}

/* orc_lut6_ffn for `batch` inputs x [batch][hidden] -> y [batch][hidden],
 * bit-identical per input; scratch holds 3 * batch * inter floats. */
void orc_lut6_ffn_batch(float* y, const uint8_t* gate_w, const uint16_t* gate_lut,
                        const uint8_t* up_w, const uint16_t* up_lut,
                        const uint8_t* down_w, const uint16_t* down_lut,
                        const float* x, int batch, int hidden, int inter, float* scratch) {
    float* g = scratch;
    float* u = scratch + (size_t)batch * inter;
    orc_lut6_matvec_batch(g, gate_w, gate_lut, x, batch, inter, hidden);
    orc_lut6_matvec_batch(u, up_w, up_lut, x, batch, inter, hidden);
    for (size_t i = 0; i < (size_t)batch * inter; i++) {
        float gv = g[i];
        g[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
    orc_lut6_matvec_batch(y, down_w, down_lut, g, batch, hidden, inter);
}

/* torch.topk over logits (scripts/export_hybrid_chunks.py:409-421) with the
 * order (value descending, index ascending); ties therefore keep the first
 * maximal index first, as the greedy rule at core/sampling.cpp:47-53 does.
 * A NaN logit ranks as -inf (the strict > of sampling.cpp:49-51 never picks a
 * NaN past index 0). */
void orc_topk(int32_t* idx, float* val, const float* logits, long n, int k) {
    int cnt = 0;
    for (long i = 0; i < n; i++) {
        float v = logits[i];
        if (v != v) v = -INFINITY;
        if (cnt == k && !(v > val[k - 1])) continue;
        int p = (cnt < k) ? cnt : k - 1;
        if (cnt < k) cnt++;
        while (p > 0 && v > val[p - 1]) {
            val[p] = val[p - 1];
            idx[p] = idx[p - 1];
            p--;
        }
        val[p] = v;
        idx[p] = (int32_t)i;
    }
}

/* core/sampling.cpp:47-53: first index of the maximum */
int orc_argmax(const float* logits, int n) {
    int m = 0;
    for (int i = 1; i < n; i++) if (logits[i] > logits[m]) m = i;
    return m;
}

/* models/llm/qwen3_5.cpp:849-908 (forward_deltanet_from_proj, norm-fused
 * first-projection layout, :853-860): proj = [mixed_qkv | z | a | b] with
 * mixed_qkv = 2*Hk*dk + Hv*dv channels, z [Hv][dv], a, b [Hv].
 * conv1d_update over mixed_qkv with the layer's ring state (:867-868), SiLU
 * (:869, silu_vec_inplace), the Q | K | V split (:872-874), then the per-head
 * recurrence and the gated norm of orc_deltanet_decode (:876-908). */
void orc_deltanet_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                            const float* proj, const float* conv_w, const float* A,
                            const float* dt_bias, const float* norm_w,
                            int Hk, int Hv, int dk, int dv, int kernel_size, int flags) {
    int qkv = 2 * Hk * dk + Hv * dv;
    float* co = (float*)malloc(sizeof(float) * (size_t)qkv);
    orc_conv1d_update(co, conv_state, conv_pos, proj, conv_w, qkv, kernel_size);
    orc_silu_vec_inplace(co, qkv);
    const float* z = proj + qkv;
    const float* a = z + (long)Hv * dv;
    const float* b = a + Hv;
    orc_deltanet_decode(y, state, co, co + (long)Hk * dk, co + 2L * Hk * dk, a, b, A, dt_bias,
                        z, norm_w, Hk, Hv, dk, dv, flags);
    free(co);
}

/* core/sampling.cpp:11-66 (sample_token) with the uniform draw r passed in
 * (the reference draws it with drand48(), :55).  Penalties over the last
 * repetition_context_size tokens of recent[0..n_recent): each distinct token
 * in range once -- repetition penalty (divide positive / multiply
 * non-positive logits) if > 1, then minus frequency_penalty * count if > 0
 * (:18-44).  temperature <= 0: first index of the maximum (:46-53).  Else
 * logits * (1/T), softmax, and the first index whose running fp32 sum reaches
 * r; vocab-1 if none (:55-66).  `adjusted` receives the penalised (and, with
 * sampling, softmax) values. */
int orc_sample_token(float* adjusted, const float* logits, int vocab, const int32_t* recent,
                     int n_recent, float temperature, float repetition_penalty,
                     int repetition_context_size, float frequency_penalty, float r) {
    memcpy(adjusted, logits, sizeof(float) * (size_t)vocab);
    if (n_recent > 0) {
        int start = n_recent - repetition_context_size;
        if (start < 0) start = 0;
        for (int j = start; j < n_recent; j++) {
            int tok = recent[j];
            if (tok < 0 || tok >= vocab) continue;
            int seen = 0, count = 0;
            for (int i = start; i < n_recent; i++) {
                if (recent[i] == tok) {
                    if (i < j) seen = 1;
                    count++;
                }
            }
            if (seen) continue;   /* one adjustment per distinct token */
            if (repetition_penalty > 1.0f) {
                if (adjusted[tok] > 0.0f) adjusted[tok] = adjusted[tok] / repetition_penalty;
                else adjusted[tok] = adjusted[tok] * repetition_penalty;
            }
            if (frequency_penalty > 0.0f) adjusted[tok] = adjusted[tok] - frequency_penalty * (float)count;
        }
    }
    if (temperature <= 0.0f) return orc_argmax(adjusted, vocab);
    float inv_t = 1.0f / temperature;
    for (int i = 0; i < vocab; i++) adjusted[i] = adjusted[i] * inv_t;
    orc_softmax(adjusted, vocab);
    float cum = 0.0f;
    for (int i = 0; i < vocab; i++) {
        cum += adjusted[i];
        if (cum >= r) return i;
    }
    return vocab - 1;
}
