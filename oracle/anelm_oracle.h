/*
 * anelm_oracle.h -- CPU restatement of ANE-LM's core/cpu_ops hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the reference the HIP kernels are
 * tested against:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product path (ane-lm_amd/libanelm.so) never links or calls it.
 *
 * Every function states the reference file:line it follows.  The reference's
 * cpu_ops.cpp calls Apple Accelerate (vDSP / vForce / CBLAS) whose internal
 * summation order is not published; the restatement uses plain sequential
 * fp32 loops, which is the mathematical definition of those routines.
 *
 * Composite functions (attention decode step, DeltaNet step, causal prefill,
 * LUT6 matvec, top-k) are compositions of the cpu_ops restatement, following
 * the caller glue in models/llm/qwen3_5.cpp.
 */
#ifndef ANELM_ORACLE_H
#define ANELM_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fp16 <-> fp32 (IEEE binary16, round-to-nearest-even) ---- */
float    orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_f16(float f);
void     orc_f16_to_f32_array(float* out, const uint16_t* in, long n);
void     orc_f32_to_f16_array(uint16_t* out, const float* in, long n);

/* ---- cpu_ops restatement (core/cpu_ops.{h,cpp}) ---- */
void orc_silu_vec_inplace(float* x, int n);
void orc_mul_sigmoid_inplace(float* y, const float* z, int n);
void orc_rmsnorm(float* out, const float* x, const float* w, int dim, float eps);
void orc_rmsnorm_gated(float* out, const float* x, const float* z, const float* w, int dim);
/* rope_mode 0 = interleaved pairs (cpu_ops), 1 = half-split (serve_hybrid / HF) */
void orc_apply_rope(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                    int q_head_stride, int k_head_stride, int rot_dim, int pos, float theta,
                    const float* cos_row, const float* sin_row, int rope_mode);
void orc_rope_table(float* cos_tab, float* sin_tab, int max_pos, int rot_dim, float theta);
void orc_softmax(float* x, int n);
void orc_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim);
void orc_l2_normalize(float* x, int dim);
void orc_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                       const float* w, int channels, int kernel_size);
/* order 0 = cpu_ops (retrieve before decay), 1 = transformers (decay first) */
void orc_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                  float decay, float beta, int key_dim, int value_dim, int order);
void orc_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                       int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                       int cache_start, int cache_len, int cache_capacity);

/* ---- compositions ---- */

/* One full-attention decode step over an fp16 ring KV cache [cap][Hkv][D].
 * q_gate [Hq][2D] (q || gate per head) and k [Hkv][D] are normalised and
 * rotated in place; v [Hkv][D].  *cache_start / *cache_len are advanced like
 * the KVCache ring.  out [Hq][D]. */
void orc_full_attn_decode(float* out, float* q_gate, float* k, const float* v,
                          uint16_t* k_cache, uint16_t* v_cache,
                          const float* q_norm_w, const float* k_norm_w,
                          int n_heads, int n_kv_heads, int head_dim, int rot_dim,
                          int pos, float theta, float eps, int rope_mode, int gate,
                          int* cache_start, int* cache_len, int cache_capacity);

/* One Gated-DeltaNet decode step for all value heads (post conv/SiLU inputs).
 * q,k [Hk][dk] are l2-normalised (if flags&1) and q scaled in place.
 * flags: 1 = l2norm q/k, 2 = transformers order, 4 = rmsnorm_gated epilogue
 * (needs z [Hv][dv] and norm_w [dv]).  y [Hv][dv]; state [Hv][dk][dv]. */
void orc_deltanet_decode(float* y, float* state, float* q, float* k, const float* v,
                         const float* a, const float* b, const float* A, const float* dt_bias,
                         const float* z, const float* norm_w,
                         int Hk, int Hv, int dk, int dv, int flags);

/* Causal prefill attention = row t attends keys 0..t (T x gqa_attention).
 * q [S][Hq][D], k/v [S][Hkv][D] fp16; out rows [row_begin,row_end) fp32. */
void orc_prefill_attention(float* out, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                           int S, int Hq, int Hkv, int D, int row_begin, int row_end);

/* Chunked-prefill semantics = sequential DeltaNet steps over S tokens.
 * q,k [S][Hk][dk] (modified in place by normalisation), v [S][Hv][dv],
 * a,b [S][Hv]; y [S][Hv][dv]; state [Hv][dk][dv] updated. */
void orc_deltanet_prefill(float* y, float* state, float* q, float* k, const float* v,
                          const float* a, const float* b, const float* A, const float* dt_bias,
                          int S, int Hk, int Hv, int dk, int dv, int flags);

/* ---- LUT6 ---- */
void orc_lut6_pack(uint8_t* packed, const uint8_t* idx, long n);
void orc_lut6_unpack(uint8_t* idx, const uint8_t* packed, long n);
void orc_lut6_dequant_row(float* w, const uint8_t* packed_row, const uint16_t* lut64, int in_dim);
void orc_lut6_matvec(float* y, const uint8_t* packed, const uint16_t* lut, const float* x,
                     int out_dim, int in_dim, int row_begin, int row_end);
void orc_lut6_matvec_batch(float* y, const uint8_t* packed, const uint16_t* lut, const float* x,
                           int batch, int out_dim, int in_dim);
void orc_lut6_ffn_batch(float* y, const uint8_t* gate_w, const uint16_t* gate_lut,
                        const uint8_t* up_w, const uint16_t* up_lut,
                        const uint8_t* down_w, const uint16_t* down_lut,
                        const float* x, int batch, int hidden, int inter, float* scratch);
void orc_lut6_ffn(float* y, const uint8_t* gate_w, const uint16_t* gate_lut,
                  const uint8_t* up_w, const uint16_t* up_lut,
                  const uint8_t* down_w, const uint16_t* down_lut,
                  const float* x, int hidden, int inter, float* scratch);
void orc_topk(int32_t* idx, float* val, const float* logits, long n, int k);
int  orc_argmax(const float* logits, int n);

/* models/llm/qwen3_5.cpp:849-908: conv1d ring + SiLU + split of the norm-fused
 * first projection proj = [mixed_qkv | z | a | b], then orc_deltanet_decode.
 * conv_state [2*Hk*dk + Hv*dv][kernel_size-1] and *conv_pos advance. */
void orc_deltanet_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                            const float* proj, const float* conv_w, const float* A,
                            const float* dt_bias, const float* norm_w,
                            int Hk, int Hv, int dk, int dv, int kernel_size, int flags);

/* core/sampling.cpp:11-66 with the uniform draw r given; returns the token. */
int orc_sample_token(float* adjusted, const float* logits, int vocab, const int32_t* recent,
                     int n_recent, float temperature, float repetition_penalty,
                     int repetition_context_size, float frequency_penalty, float r);

#ifdef __cplusplus
}
#endif
#endif
