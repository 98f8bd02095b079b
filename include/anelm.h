/*
 * anelm.h -- C ABI of libanelm.so, the MI355X (gfx950) implementation of the
 * ANE-LM core/cpu_ops hot path.
 *
 * Native tier: every pointer argument is a DEVICE pointer unless marked
 * "host"; `stream` is a hipStream_t passed as void* (NULL = null stream).
 * Calls are asynchronous on `stream` and return an int status:
 *   0 = ANELM_OK, < 0 = error (see anelm_last_error(), thread-local text).
 * Nothing throws across the ABI.  Device scratch (workspaces and the zeroed
 * counters of in-kernel reductions) is owned per (device, stream): calls on
 * different streams share no mutable state and may run concurrently, from
 * one host thread or several, as the reference's cpu_ops functions keep no
 * mutable globals (core/cpu_ops.cpp:1-206).  Calls on one stream are ordered
 * by that stream; one host thread at a time may issue on a given stream.
 * anelm_stream_release frees a stream's scratch before the stream is
 * destroyed.
 *
 * Each declaration names the reference interface it replaces.
 */
#ifndef ANELM_H
#define ANELM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    ANELM_OK = 0,
    ANELM_EINVAL = -1,   /* bad shape, stride or flag */
    ANELM_ENULL = -2,    /* required pointer is NULL */
    ANELM_EHIP = -3,     /* HIP runtime error */
    ANELM_ERANGE = -4,   /* size beyond a supported maximum */
    ANELM_ENOMEM = -5    /* workspace allocation failed */
};

/* RoPE pairing: core/cpu_ops.cpp:40-63 rotates interleaved pairs (v[i], v[i+1]);
 * scripts/serve_hybrid.py:94-103 rotates (v[j], v[j + rot/2]). */
#define ANELM_ROPE_INTERLEAVED 0
#define ANELM_ROPE_HALF_SPLIT 1

/* DeltaNet flags. */
#define ANELM_DN_L2NORM 1              /* l2-normalise q,k per key head (qwen3_5.cpp:882-887) */
#define ANELM_DN_ORDER_TRANSFORMERS 2  /* decay-first rule (export_hybrid_chunks.py:137-147) */
#define ANELM_DN_GATED_NORM 4          /* rmsnorm_gated epilogue (qwen3_5.cpp:902-908) */

/* Cache element types. */
#define ANELM_F32 0
#define ANELM_F16 1

/* KV cache layouts: the reference's token-major ring [capacity][Hkv][D]
 * (models/llm/qwen3_5.cpp:335-336) and the head-major cache [Hkv][ctx][D] of
 * scripts/serve_hybrid.py:232-235. */
#define ANELM_KV_TOKEN_MAJOR 0
#define ANELM_KV_HEAD_MAJOR 1

const char* anelm_last_error(void);
int anelm_version(void);
/* Number of compute units of the current device (0 on error). */
int anelm_device_cus(void);
/* Frees the library's scratch for `stream` on the current device (created
 * by the first call on that stream), after waiting for the stream.  Call it
 * before destroying a stream that library calls were issued on.  No
 * counterpart in the reference (its functions use alloca / malloc per call,
 * core/cpu_ops.cpp:35, 165, 203). */
int anelm_stream_release(void* stream);

/* ---------------------------------------------------------------- norms */

/* rmsnorm, core/cpu_ops.h:21 / cpu_ops.cpp:24-30, over n_rows rows of `dim`
 * (row r of x at x + r*x_stride, of out at out + r*out_stride).  In place is
 * allowed (out == x with equal strides). */
int anelm_rmsnorm(float* out, const float* x, const float* weight, int dim, int n_rows,
                  int x_stride, int out_stride, float eps, void* stream);

/* rmsnorm_gated, cpu_ops.h:22 / cpu_ops.cpp:32-38, per row:
 * out = rmsnorm(x, w, 1e-6) * sigmoid(z) * z. */
int anelm_rmsnorm_gated(float* out, const float* x, const float* z, const float* weight,
                        int dim, int n_rows, void* stream);

/* l2_normalize, cpu_ops.h:41 / cpu_ops.cpp:82-87, in place per row. */
int anelm_l2_normalize(float* x, int dim, int n_rows, void* stream);

/* ----------------------------------------------------------------- RoPE */

/* apply_rope_cached, cpu_ops.h:26-29 / cpu_ops.cpp:40-63.  cos_row/sin_row
 * are HOST pointers to rot_dim/2 floats (the qwen3_5.cpp:308-324 table row)
 * or NULL, in which case cosf/sinf(pos * theta^(-i/rot_dim)) are evaluated on
 * the host exactly as cpu_ops.cpp:51-55 does.  rot_dim <= 256, even. */
int anelm_apply_rope(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                     int q_head_stride, int k_head_stride, int rot_dim, int pos, float theta,
                     const float* cos_row, const float* sin_row, int rope_mode, void* stream);

/* ------------------------------------------------------------ activations */

/* silu_vec_inplace (cpu_ops.cpp:6-13) and mul_sigmoid_inplace (:15-22); the
 * reference's caller-provided tmp scratch is not needed. */
int anelm_silu_inplace(float* x, int n, void* stream);
int anelm_mul_sigmoid_inplace(float* y, const float* z, int n, void* stream);

/* softmax, cpu_ops.h:33 / cpu_ops.cpp:65-75, in place over n_rows rows of n. */
int anelm_softmax(float* x, int n, int n_rows, void* stream);

/* matvec, cpu_ops.h:37 / cpu_ops.cpp:77-80: y = W x, W row-major fp32. */
int anelm_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim, void* stream);

/* conv1d_update, cpu_ops.h:45-46 / cpu_ops.cpp:89-129.  conv_state is a device
 * array [channels][kernel_size-1]; *state_pos is a HOST int advanced here. */
int anelm_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                        const float* w, int channels, int kernel_size, void* stream);

/* ------------------------------------------------------------ attention */

/* gqa_attention, cpu_ops.h:55-58 / cpu_ops.cpp:148-204, over a ring cache
 * [cache_capacity][n_kv_heads][head_dim] of fp32 (kv_dtype ANELM_F32, the
 * reference layout) or fp16 (ANELM_F16).  Keys are taken oldest to newest from
 * cache_start; cache_len <= 0 writes zeros (cpu_ops.cpp:152-155).
 * head_dim in {64, 128, 256}; n_heads / n_kv_heads in {1, 2, 4, 8}. */
int anelm_gqa_attention(float* out, const float* q, const void* k_cache, const void* v_cache,
                        int kv_dtype, int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                        int cache_start, int cache_len, int cache_capacity, void* stream);

/* One full-attention decode step, the composition at
 * models/llm/qwen3_5.cpp:944-1002, fused into one launch:
 *   per-head RMSNorm of q (rows of q_gate, stride 2*head_dim) and k with
 *   q_norm_w / k_norm_w (:952-959); RoPE (:961-971); fp16 ring append of k, v
 *   (:973-986); gqa_attention (:989-991); sigmoid output gate when `gate`
 *   (:993-1000).
 * q_norm_w and k_norm_w may both be NULL: no q/k RMSNorm, for callers that
 * receive normalised q/k (scripts/serve_hybrid.py:89-107 applies RoPE only).
 * q_gate [n_heads][2*head_dim], k/v [n_kv_heads][head_dim] are read only.
 * *cache_start / *cache_len are HOST ints advanced as the KVCache ring does.
 * cos_row/sin_row: HOST, as for anelm_apply_rope. */
int anelm_full_attn_decode(float* out, const float* q_gate, const float* k, const float* v,
                           uint16_t* k_cache, uint16_t* v_cache,
                           const float* q_norm_w, const float* k_norm_w,
                           int n_heads, int n_kv_heads, int head_dim, int rot_dim,
                           int pos, float theta, float eps, int rope_mode, int gate,
                           const float* cos_row, const float* sin_row,
                           int* cache_start, int* cache_len, int cache_capacity, void* stream);

/* anelm_full_attn_decode over a cache of element type kv_dtype (ANELM_F16 or
 * ANELM_F32, the reference's fp32 cache) and layout ANELM_KV_TOKEN_MAJOR or
 * ANELM_KV_HEAD_MAJOR.  With q_norm_w = k_norm_w = NULL, rope_mode
 * ANELM_ROPE_HALF_SPLIT, a head-major fp32 cache, cache_start 0 and
 * cache_len = pos this is scripts/serve_hybrid.py:85-132 (cpu_attention):
 * RoPE at pos, k and v written at slot pos, attention over keys 0..pos,
 * sigmoid gate. */
int anelm_full_attn_decode_kv(float* out, const float* q_gate, const float* k, const float* v,
                              void* k_cache, void* v_cache, int kv_dtype, int layout,
                              const float* q_norm_w, const float* k_norm_w, int n_heads, int n_kv_heads,
                              int head_dim, int rot_dim, int pos, float theta, float eps, int rope_mode,
                              int gate, const float* cos_row, const float* sin_row, int* cache_start,
                              int* cache_len, int cache_capacity, void* stream);

/* anelm_full_attn_decode without any device allocation, for callers that
 * cannot allocate (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.  Same
 * arguments and results as anelm_full_attn_decode; the split partials live in
 * a static per-device array of 8 MiB (held by every device the library runs
 * on until the process ends), which bounds n_kv_heads * ceil(len / (256 / G))
 * * G * (head_dim + 2) * 4 bytes plus 1 KiB of split-merge counters (len =
 * keys attended after the append, G = n_heads / n_kv_heads): 16 q / 4 kv
 * heads at head_dim 256 attend up to
 * 32448 keys.  Larger calls return ANELM_ERANGE.  Calls that overlap on one
 * device share that array and race; the library's first call on a device
 * that allocates (e.g. anelm_device_cus) is not needed before this one. */
int anelm_full_attn_decode_noalloc(float* out, const float* q_gate, const float* k, const float* v,
                                   uint16_t* k_cache, uint16_t* v_cache,
                                   const float* q_norm_w, const float* k_norm_w,
                                   int n_heads, int n_kv_heads, int head_dim, int rot_dim,
                                   int pos, float theta, float eps, int rope_mode, int gate,
                                   const float* cos_row, const float* sin_row,
                                   int* cache_start, int* cache_len, int cache_capacity, void* stream);

/* Batched decode over paged fp16 caches (no reference kernel: per sequence it
 * is gqa_attention, cpu_ops.cpp:148-204, over that sequence's keys).
 * n_pages pages hold page_size tokens each as [page][n_kv_heads][page_size][head_dim].
 * Sequence s attends keys 0..min(seq_lens[s], max_seq_len)-1 (an empty
 * sequence yields zeros); key t lives in page page_table[s*max_pages + t/page_size]
 * (clamped to [0, n_pages)) at row t%page_size.
 * q [n_seqs][n_heads][q_head_stride]; out [n_seqs][n_heads][head_dim].
 * seq_lens, page_table: device int32. */
int anelm_attn_decode_paged(float* out, const float* q, int q_head_stride,
                            const uint16_t* k_pages, const uint16_t* v_pages,
                            const int32_t* page_table, const int32_t* seq_lens,
                            int n_seqs, int max_pages, int page_size, int n_pages, int max_seq_len,
                            int n_heads, int n_kv_heads, int head_dim, void* stream);

/* One full-attention decode step for a batch of sequences over paged fp16
 * caches (no reference kernel as one call): per sequence s the composition
 * of anelm_full_attn_decode, models/llm/qwen3_5.cpp:944-1002 --
 *   RMSNorm of its q rows (q_gate [n_seqs][n_heads][2*head_dim]) and k
 *   (k, v [n_seqs][n_kv_heads][head_dim]) with q_norm_w / k_norm_w (both
 *   NULL: no norm); RoPE at position positions[s] (device int32; NULL:
 *   seq_lens[s]); fp16 append of k, v as key seq_lens[s] (page
 *   page_table[s*max_pages + seq_lens[s]/page_size], row
 *   seq_lens[s] % page_size); gqa_attention (cpu_ops.cpp:148-204) over keys
 *   0..seq_lens[s]; the sigmoid output gate when `gate`.
 * seq_lens (device int32) counts each sequence's cached keys before the
 * step and is not advanced here; sequences with seq_lens[s] + 1 >
 * max_seq_len attend their first max_seq_len keys and append nothing.
 * RoPE cos/sin come from rope_table [rope_rows][rot_dim] (device; row pos =
 * cos of the rot_dim/2 pairs, then sin -- see anelm_rope_table) for
 * positions below rope_rows, else from the same formula evaluated on the
 * device (rope_table may be NULL), as qwen3_5.cpp:961-971 switches from its
 * table to cpu_ops.cpp:51-55 past 4096.  Pages as for anelm_attn_decode_paged;
 * out [n_seqs][n_heads][head_dim]. */
int anelm_attn_decode_paged_step(float* out, const float* q_gate, const float* k, const float* v,
                                 uint16_t* k_pages, uint16_t* v_pages, const int32_t* page_table,
                                 const int32_t* seq_lens, const int32_t* positions,
                                 const float* q_norm_w, const float* k_norm_w,
                                 const float* rope_table, int rope_rows,
                                 int n_seqs, int max_pages, int page_size, int n_pages, int max_seq_len,
                                 int n_heads, int n_kv_heads, int head_dim, int rot_dim, float theta,
                                 float eps, int rope_mode, int gate, void* stream);

/* RoPE table rows 0..n_pos-1 (models/llm/qwen3_5.cpp:308-324): row pos holds
 * cosf(pos * f_j) for the rot_dim/2 pairs j, then sinf(pos * f_j), with
 * f_j = 1 / powf(theta, 2j / rot_dim), evaluated on the host exactly as
 * cpu_ops.cpp:51-55 and copied to the device array `table`
 * [n_pos][rot_dim].  Synchronous. */
int anelm_rope_table(float* table, int rot_dim, int n_pos, float theta);

/* Causal GQA prefill (no reference kernel: generate.cpp:76-84 runs the
 * decode core per token, so row t attends keys 0..t).  q [S][Hq][D],
 * k/v [S][Hkv][D] fp16; out [S][Hq][D] fp32 (out_dtype ANELM_F32) or fp16.
 * head_dim 256 or 128; Hq % Hkv == 0. */
int anelm_attn_prefill(void* out, int out_dtype, const uint16_t* q, const uint16_t* k,
                       const uint16_t* v, int S, int n_heads, int n_kv_heads, int head_dim,
                       void* stream);

/* Prompt prefill through one full-attention layer core: the S decode steps
 * generate.cpp:55-85 runs for a prompt (forward_full_attn_from_proj,
 * models/llm/qwen3_5.cpp:944-1002, per token; forward_batch, :1164-1217,
 * batches only the projections around it) as one call.  Token t of the
 * prompt, at position pos0 + t:
 *   q rows (q_gate [S][n_heads][2*head_dim]) and k (k, v
 *   [S][n_kv_heads][head_dim]) RMS-normalised with q_norm_w / k_norm_w (both
 *   NULL: no norm, :952-959); RoPE at pos0 + t (:961-971); k, v appended to
 *   the fp16 ring as the t-th new key (:973-986); gqa_attention over the ring
 *   as it stands after that append -- the last min(capacity, len0 + t + 1)
 *   keys, len0 = *cache_len on entry (:989-991); the sigmoid output gate when
 *   `gate` (:993-1000).
 * proj_stride: floats from one token's rows to the next in q_gate, k and v
 * -- with the first projection's output [S][q_gate | k | v] (forward_batch's
 * proj_batch_, :1181-1189) pass q_gate = proj, k = proj + n_heads*2*head_dim,
 * v = k + n_kv_heads*head_dim and its row length; 0 = each array packed.
 * out [S][n_heads][head_dim] fp32.  *cache_start / *cache_len (HOST ints)
 * end as after S appends; prompt keys that a later prompt key overwrote are
 * not written.  RoPE rows: rope_table (device, [rope_rows][rot_dim]: cos of
 * the rot_dim/2 pairs, then sin -- anelm_rope_table, the reference's table of
 * qwen3_5.cpp:308-324) for positions below rope_rows, else the same formula
 * on the device (the reference switches to cpu_ops.cpp:51-55 past its
 * table); rope_table may be NULL.  q enters the fp16 MFMA products as fp16
 * (after norm and RoPE in fp32); keys and values are the cache's fp16.
 * head_dim 128 or 256; n_heads / n_kv_heads in {1, 2, 4, 8}. */
int anelm_full_attn_prefill(float* out, const float* q_gate, const float* k, const float* v,
                            int proj_stride, uint16_t* k_cache, uint16_t* v_cache, const float* q_norm_w,
                            const float* k_norm_w, int S, int n_heads, int n_kv_heads, int head_dim,
                            int rot_dim, int pos0, float theta, float eps, int rope_mode, int gate,
                            const float* rope_table, int rope_rows, int* cache_start, int* cache_len,
                            int cache_capacity, void* stream);

/* ------------------------------------------------------------- DeltaNet */

/* ssm_step, cpu_ops.h:50-51 / cpu_ops.cpp:131-146, for one head:
 * state [key_dim][value_dim] fp32 updated in place, y [value_dim].
 * decay and beta are scalars (HOST floats), order as ANELM_DN_ORDER_*. */
int anelm_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                   float decay, float beta, int key_dim, int value_dim, int flags, void* stream);

/* One Gated-DeltaNet decode step for all heads, the composition at
 * models/llm/qwen3_5.cpp:879-908 after conv/SiLU:
 *   q,k [Hk][dk] (read only), v [Hv][dv], a,b [Hv] projections,
 *   A [Hv] = exp(A_log) (qwen3_5.cpp:417-421), dt_bias [Hv];
 *   beta = sigmoid(b), decay = exp(-A*softplus(a+dt_bias)) (:896-898);
 *   value head h uses key head h/(Hv/Hk) (:890);
 *   state [Hv][dk][dv] fp32 updated in place; y [Hv][dv];
 *   with ANELM_DN_GATED_NORM, y = rmsnorm_gated(y, z [Hv][dv], norm_w [dv]).
 * dk, dv = 128. */
int anelm_deltanet_decode(float* y, float* state, const float* q, const float* k, const float* v,
                          const float* a, const float* b, const float* A, const float* dt_bias,
                          const float* z, const float* norm_w,
                          int Hk, int Hv, int dk, int dv, int flags, void* stream);

/* anelm_deltanet_decode for n_seqs sequences in one launch: each sequence
 * has its own inputs and state -- q,k [n_seqs][Hk][dk], v, z, y
 * [n_seqs][Hv][dv], a,b [n_seqs][Hv], state [n_seqs][Hv][dk][dv] -- and
 * shares the layer weights A, dt_bias [Hv] and norm_w [dv].  Per sequence
 * the same composition as anelm_deltanet_decode (qwen3_5.cpp:879-908);
 * n_seqs * Hv <= 65535. */
int anelm_deltanet_decode_batched(float* y, float* state, const float* q, const float* k, const float* v,
                                  const float* a, const float* b, const float* A, const float* dt_bias,
                                  const float* z, const float* norm_w,
                                  int n_seqs, int Hk, int Hv, int dk, int dv, int flags, void* stream);

/* Qwen35Model::forward_deltanet_from_proj (models/llm/qwen3_5.cpp:849-908) in
 * one launch: conv1d_update + SiLU (cpu_ops.cpp:89-129, :6-13) over the
 * mixed q|k|v channels of the norm-fused first projection, the Q | K | V
 * split, then the composition of anelm_deltanet_decode.
 *   proj = [mixed_qkv (2*Hk*dk + Hv*dv) | z (Hv*dv) | a (Hv) | b (Hv)];
 *   conv_state [2*Hk*dk + Hv*dv][conv_kernel-1] device ring, conv_w
 *   [2*Hk*dk + Hv*dv][conv_kernel]; *conv_pos is a HOST int advanced here
 *   (the reference's DeltaNetState::conv_pos, qwen3_5.h:158-162).
 * Flags as anelm_deltanet_decode; dk, dv = 128. */
int anelm_deltanet_decode_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                                    const float* proj, const float* conv_w, const float* A,
                                    const float* dt_bias, const float* norm_w, int Hk, int Hv,
                                    int dk, int dv, int conv_kernel, int flags, void* stream);

/* Chunked DeltaNet prefill over S tokens (no reference kernel: the reference
 * runs ssm_step per token, qwen3_5.cpp:1204-1217).  q,k [S][Hk][dk],
 * v [S][Hv][dv], a,b [S][Hv]; y [S][Hv][dv]; state [Hv][dk][dv] updated to the
 * state after token S-1.  chunk = 64: chunked closed form (per 64-token chunk
 * the state-independent products in parallel, then the state carried through
 * the chunks); chunk = 1: token-by-token scan.  Flags as anelm_deltanet_decode minus
 * GATED_NORM.  dk, dv = 128. */
int anelm_deltanet_prefill(float* y, float* state, const float* q, const float* k, const float* v,
                           const float* a, const float* b, const float* A, const float* dt_bias,
                           int S, int Hk, int Hv, int dk, int dv, int chunk, int flags, void* stream);

/* Prompt prefill through one Gated-DeltaNet layer core from its projections:
 * the S steps of anelm_deltanet_decode_from_proj (forward_deltanet_from_proj,
 * models/llm/qwen3_5.cpp:849-908, per token, as generate.cpp:55-85 and
 * forward_batch :1164-1217 run it over a prompt) as one call.
 *   proj [S][2*Hk*dk + Hv*dv + Hv*dv + 2*Hv]: per token [mixed qkv | z | a | b];
 *   the causal conv1d over the conv ring followed by the prompt's mixed
 *   channels + SiLU (cpu_ops.cpp:89-129, :6-13), split into q | k | v; the
 *   chunked recurrence (anelm_deltanet_prefill); with ANELM_DN_GATED_NORM,
 *   rmsnorm_gated(y, z, norm_w) per token and value head (:902-908).
 * y [S][Hv][dv]; state [Hv][dk][dv] ends after the last token; conv_state
 * [2*Hk*dk + Hv*dv][conv_kernel-1] and *conv_pos (HOST int) end as after S
 * conv1d_update calls.  dk, dv = 128; conv_kernel 2..16. */
int anelm_deltanet_prefill_from_proj(float* y, float* state, float* conv_state, int* conv_pos,
                                     const float* proj, const float* conv_w, const float* A,
                                     const float* dt_bias, const float* norm_w, int S, int Hk, int Hv,
                                     int dk, int dv, int conv_kernel, int flags, void* stream);

/* ----------------------------------------------------------------- LUT6 */
/* LUT6 weight format: W[r][c] = lut[r/32][idx(r,c)], lut fp16 [out/32][64],
 * idx 6-bit, row-major, row r at w + r*in_dim*3/4 bytes, index c at bits
 * [6c, 6c+6) of the little-endian row stream (4 indices per 3 bytes).
 * out_dim % 32 == 0, in_dim % 16 == 0. */

/* Unpack n (multiple of 4) indices to one byte each. */
int anelm_lut6_unpack(uint8_t* idx, const uint8_t* packed, int64_t n, void* stream);

/* y = W x (matvec, cpu_ops.cpp:77-80, on the dequantised weights). */
int anelm_lut6_gemv(float* y, const uint8_t* w, const uint16_t* lut, const float* x,
                    int out_dim, int in_dim, void* stream);

/* A layer projection around the cores on LUT6 weights: y = W n, or y += W n
 * with accumulate (the residual add of o_proj, qwen3_5.cpp:1310-1327), where
 * n = rmsnorm(x, norm_w, eps) (the input norm fused into the first
 * projection, :1287-1300, 1004-1011) or x when norm_w is NULL.  The
 * activations enter the dot products as fp16, as in anelm_lut6_gemv. */
int anelm_lut6_proj(float* y, const uint8_t* w, const uint16_t* lut, const float* x, const float* norm_w,
                    float eps, int out_dim, int in_dim, int accumulate, void* stream);

/* SwiGLU FFN block with residual (qwen3_5.cpp:1335-1354 with the MLP of
 * :1118-1130): n = rmsnorm(x, norm_w, eps) (skipped when norm_w is NULL);
 * x += down( silu(gate n) * (up n) ).  x [hidden] is updated in place;
 * gu_scratch [2*inter] is scratch: its first inter entries receive
 * h = silu(gate n) * (up n), the rest is undefined. */
int anelm_lut6_ffn(float* x, float* gu_scratch, const float* norm_w, float eps,
                   const uint8_t* gate_w, const uint16_t* gate_lut,
                   const uint8_t* up_w, const uint16_t* up_lut,
                   const uint8_t* down_w, const uint16_t* down_lut,
                   int hidden, int inter, void* stream);

/* The two projections of the FFN block (qwen3_5.cpp:1118-1122):
 * g = gate n, u = up n, n = rmsnorm(x, norm_w, eps) (x when norm_w is NULL).
 * One launch over both matrices.  g, u [inter]. */
int anelm_lut6_gate_up(float* g, float* u, const float* x, const float* norm_w, float eps,
                       const uint8_t* gate_w, const uint16_t* gate_lut,
                       const uint8_t* up_w, const uint16_t* up_lut,
                       int hidden, int inter, void* stream);

/* The gate/up half of the FFN block alone (qwen3_5.cpp:1118-1126):
 * h = silu(gate n) * (up n), n = rmsnorm(x, norm_w, eps) (x when norm_w is
 * NULL).  x [hidden], h [inter]. */
int anelm_lut6_swiglu(float* h, const float* x, const float* norm_w, float eps,
                      const uint8_t* gate_w, const uint16_t* gate_lut,
                      const uint8_t* up_w, const uint16_t* up_lut,
                      int hidden, int inter, void* stream);

/* Batched LUT6 projection: y[b] = W x[b] (accumulate = 0) or y[b] += W x[b]
 * (accumulate = 1, e.g. the residual add after the FFN down projection) for
 * b < batch (x [batch][in_dim], y [batch][out_dim], fp32; x enters the
 * products as fp16, as in anelm_lut6_gemv).  Each weight is dequantised once
 * per 32 inputs.  No reference counterpart as one call: matvec
 * (core/cpu_ops.cpp:77-80) per input on the dequantised weights. */
int anelm_lut6_gemm(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int batch,
                    int out_dim, int in_dim, int accumulate, void* stream);

/* h[i] = silu(g[i]) * u[i] for i < n -- the SwiGLU product of the FFN
 * (models/llm/qwen3_5.cpp:1118-1130) on batched gate / up outputs. */
int anelm_swiglu(float* h, const float* g, const float* u, int64_t n, void* stream);

/* h[r][i] = silu(gu[r][i]) * gu[r][n + i] for r < rows, i < n: SwiGLU over the
 * output of one projection that holds the gate rows then the up rows (a
 * batched FFN computes gate and up in one anelm_lut6_gemm over the stacked
 * [gate; up] weights).  Replaces qwen3_5.cpp:1123-1126 per row. */
int anelm_swiglu_rows(float* h, const float* gu, int rows, int n, void* stream);

/* Top-k of logits = W x for a batch of inputs (in-model top-k LM head,
 * scripts/export_hybrid_chunks.py:409-421).  x [batch][in_dim] fp32;
 * out_idx / out_val [batch][k], ordered by (value desc, index asc), so
 * out_idx[b*k] is the greedy token of core/sampling.cpp:47-53.  k <= 64. */
int anelm_lut6_topk(int32_t* out_idx, float* out_val, const uint8_t* w, const uint16_t* lut,
                    const float* x, int batch, int out_dim, int in_dim, int k, void* stream);

/* ------------------------------------------------------------- sampling */

/* sample_token, core/sampling.h:15-17 / sampling.cpp:11-66, on device logits
 * [vocab]: penalties of the distinct tokens among the last
 * repetition_context_size entries of recent [n_recent] (device int32;
 * repetition penalty if > 1, frequency penalty * count if > 0), then
 * temperature <= 0: the first index of the maximum; else softmax(logits / T)
 * and the first index whose running sum reaches r, or vocab-1.  r is the
 * uniform draw in [0, 1) the reference takes from drand48() (:57): the caller
 * owns the random stream.  *token (device int32) receives the result; logits
 * are not modified (the adjusted copy lives in the library workspace).
 * At most 4096 tokens in the penalty window.  Greedy: a NaN logit never
 * becomes the maximum, but a NaN at index 0 returns 0, as the reference's
 * scan from max_i = 0 with a strict > does (sampling.cpp:47-53). */
int anelm_sample_token(int32_t* token, const float* logits, int vocab, const int32_t* recent,
                       int n_recent, float temperature, float repetition_penalty,
                       int repetition_context_size, float frequency_penalty, float r, void* stream);

/* ------------------------------------------------- hybrid decode step */
/* The layer loop of Qwen35Model::forward (models/llm/qwen3_5.cpp:1278-1356)
 * over the compute cores: per layer the DeltaNet core (:849-910) or the
 * full-attention core (:944-1002), then the FFN block with residual
 * (:1335-1354).  The projections around the cores (first_proj, o_proj) are
 * not part of it: each layer's core reads its own input buffers and writes
 * core_out; the FFN chain carries the hidden state x from layer to layer.
 * Layer kinds follow qwen3_5.cpp:64-71. */
#define ANELM_LAYER_DELTANET 0
#define ANELM_LAYER_ATTENTION 1

typedef struct {
    int kind;
    /* full-attention core (kind ANELM_LAYER_ATTENTION) */
    const float* q_gate;        /* [Hq][2D] */
    const float* k;             /* [Hkv][D] */
    const float* v;
    uint16_t* k_cache;          /* fp16 ring [cap][Hkv][D] */
    uint16_t* v_cache;
    const float* q_norm_w;
    const float* k_norm_w;
    int cache_start, cache_len, cache_capacity, pos;
    /* DeltaNet core (kind ANELM_LAYER_DELTANET), flags as anelm_deltanet_decode */
    float* state;               /* [Hv][dk][dv] */
    const float* dn_q;          /* [Hk][dk] */
    const float* dn_k;
    const float* dn_v;          /* [Hv][dv] */
    const float* dn_a;
    const float* dn_b;
    const float* dn_A;
    const float* dn_dt_bias;
    const float* dn_z;          /* [Hv][dv] or NULL (no gated norm) */
    const float* dn_norm_w;
    int dn_flags;
    float* core_out;            /* [Hq*D] or [Hv*dv] */
    /* FFN block: x += down(silu(gate n) * (up n)), n = rmsnorm(x, ffn_norm_w) */
    const float* ffn_norm_w;
    const uint8_t* gate_w;
    const uint16_t* gate_lut;
    const uint8_t* up_w;
    const uint16_t* up_lut;
    const uint8_t* down_w;
    const uint16_t* down_lut;
    /* Projections around the core (qwen3_5.cpp:1287-1327).  first_w NULL:
     * the core inputs above are given and the layer is core + FFN.  With
     * them the layer is the whole of qwen3_5.cpp:1287-1354:
     *   proj = first_w rmsnorm(x, in_norm_w) -- DeltaNet [mixed qkv | z | a | b]
     *   (:849-860), attention [q_gate | k | v] (:948-950);
     *   the core from proj (DeltaNet through the conv ring, :867-874; the
     *   dn_q..dn_z / q_gate, k, v pointers are ignored);
     *   x += o_w core_out (:1310-1323); then the FFN block.
     * Eager runs advance conv_pos with the rings. */
    const float* in_norm_w;      /* [hidden] (NULL: no input norm) */
    const uint8_t* first_w;      /* LUT6 [first_out][hidden] */
    const uint16_t* first_lut;
    const uint8_t* o_w;          /* LUT6 [hidden][Hq*D or Hv*dv] */
    const uint16_t* o_lut;
    float* proj;                 /* scratch [first_out] */
    float* conv_state;           /* DeltaNet [2*Hk*dk + Hv*dv][conv_kernel-1] */
    const float* conv_w;         /* DeltaNet [2*Hk*dk + Hv*dv][conv_kernel] */
    int conv_pos;
} anelm_hybrid_layer;

typedef struct {
    int hidden, inter;
    int n_heads, n_kv_heads, head_dim, rot_dim, rope_mode;
    float theta, eps;
    int lin_k_heads, lin_v_heads, lin_dim;
    int conv_kernel;             /* DeltaNet conv1d width (qwen3_5.h: 4); used with projections */
} anelm_hybrid_dims;

typedef struct anelm_hybrid_step anelm_hybrid_step;

/* Execution modes of a step (the `mode` argument):
 *   ANELM_STEP_EAGER       one launch per kernel; each run advances every
 *                          attention ring and position by one token, as the
 *                          model's decode loop does;
 *   ANELM_STEP_GRAPH       the eager launches captured once into a HIP graph on
 *                          `stream` (not the null stream) at create (no step
 *                          runs then; the step owns the attention layers'
 *                          split-partial buffers, so later calls that grow the
 *                          library workspace cannot invalidate the graph);
 *                          each run replays the same work (rings do not
 *                          advance);
 *   ANELM_STEP_PERSISTENT  the whole step as ONE kernel launch (one workgroup
 *                          per compute unit, grid barriers between the
 *                          layers' phases); advances rings like EAGER (the
 *                          launch writes the next step's ring descriptors
 *                          itself: consecutive runs queue without a host
 *                          wait, except once per 4096 positions when the
 *                          RoPE table grows), or replays like GRAPH when
 *                          combined with ANELM_STEP_STATIC.  Supported for hidden/inter
 *                          sizes that tile over the device's compute units
 *                          (the Qwen3.5-4B and Qwen3.5-0.8B shapes on 256
 *                          CUs) and core + FFN layers (first_w NULL); other
 *                          shapes, and complete layers (disabled), return
 *                          ANELM_EINVAL from create.
 *   ANELM_STEP_COOPERATIVE (with PERSISTENT) launches through
 *                          hipLaunchCooperativeKernel: the runtime starts the
 *                          grid only when every workgroup can be resident, so
 *                          kernels running concurrently on other streams delay
 *                          the step instead of starving its grid barriers
 *                          (without it, such a step gives up after ~0.7 s and
 *                          reports status 1).  Costs ~17 us per step on
 *                          MI355X. */
#define ANELM_STEP_EAGER 0
#define ANELM_STEP_GRAPH 1
#define ANELM_STEP_PERSISTENT 2
#define ANELM_STEP_STATIC 4
#define ANELM_STEP_COOPERATIVE 8

/* Builds a step over n_layers descriptors (copied), x [hidden] and
 * h_scratch [2*inter] device buffers (the step's FFN scratch). */
int anelm_hybrid_step_create(anelm_hybrid_step** out, const anelm_hybrid_dims* dims,
                             const anelm_hybrid_layer* layers, int n_layers, float* x,
                             float* h_scratch, int mode, void* stream);
int anelm_hybrid_step_run(anelm_hybrid_step* step, void* stream);
/* Synchronous: *status = 0 if every persistent run so far completed, 1 if a
 * run gave up waiting at a grid barrier (its outputs are then invalid);
 * clears the flag.  Always 0 for the eager and graph modes. */
int anelm_hybrid_step_status(anelm_hybrid_step* step, int* status);
/* Diagnostic (no counterpart in the reference): copies the phase timeline of
 * the last persistent run to host memory -- per workgroup, per phase
 * (3 per layer: core, gate/up, down; then one row of kernel entry/exit),
 * eight 100 MHz real-time clock stamps: compute start, compute end, barrier
 * arrival, barrier release observed, then (GEMV phases) first weight issue
 * done, pair tables built, early lookups done, second weight issue done.  Only libanelm_trace.so (the same
 * library built with ANELM_STEP_TRACE=1) records it; libanelm.so returns
 * ANELM_EINVAL.  *grid and *phases receive the buffer's dimensions. */
int anelm_hybrid_step_trace(anelm_hybrid_step* step, uint64_t* host, size_t n_words, int* grid,
                            int* phases);
int anelm_hybrid_step_destroy(anelm_hybrid_step* step);

/* ------------------------------------------------ batched decode step */
/* The layer loop of Qwen35Model::forward (models/llm/qwen3_5.cpp:1278-1356)
 * over the compute cores for n_seqs concurrent sequences (the JSON-lines
 * serve loop, main.cpp:241-377, serves them one at a time): per layer the
 * full-attention core over every sequence's paged cache
 * (anelm_attn_decode_paged_step) or the DeltaNet core over every
 * sequence's state (anelm_deltanet_decode_batched), then the SwiGLU FFN
 * block with residual on x [n_seqs][hidden] through the batched LUT6
 * projection (each weight dequantised once per 32 sequences); optionally
 * the final norm and the top-k of the LUT6 LM head.  Per-sequence inputs
 * carry a leading [n_seqs] dimension. */
typedef struct {
    int kind;                     /* ANELM_LAYER_* */
    /* full attention */
    const float* q_gate;          /* [B][Hq][2D] */
    const float* k;               /* [B][Hkv][D] */
    const float* v;
    uint16_t* k_pages;            /* [n_pages][Hkv][page_size][D] fp16, this layer's pool */
    uint16_t* v_pages;
    const int32_t* page_table;    /* [B][max_pages] */
    const float* q_norm_w;        /* [D] (both NULL: no q/k norm) */
    const float* k_norm_w;
    /* DeltaNet */
    float* state;                 /* [B][Hv][dk][dv] */
    const float* dn_q;            /* [B][Hk][dk] */
    const float* dn_k;
    const float* dn_v;            /* [B][Hv][dv] */
    const float* dn_a;            /* [B][Hv] */
    const float* dn_b;
    const float* dn_A;            /* [Hv], exp(A_log) */
    const float* dn_dt_bias;      /* [Hv] */
    const float* dn_z;            /* [B][Hv][dv] (gated norm) */
    const float* dn_norm_w;       /* [dv] */
    int dn_flags;
    float* core_out;              /* [B][Hq*D] or [B][Hv*dv] */
    /* FFN */
    const float* ffn_norm_w;      /* [hidden] */
    const uint8_t* gate_up_w;     /* LUT6 [2*inter][hidden]: the gate rows, then the up rows */
    const uint16_t* gate_up_lut;  /* [2*inter/32][64] */
    const uint8_t* down_w;        /* LUT6 [hidden][inter] */
    const uint16_t* down_lut;
} anelm_batch_layer;

typedef struct {
    int n_seqs;
    int32_t* seq_lens;            /* device [B]: cached keys per sequence */
    int32_t* positions;           /* device [B]: position of each new token, or NULL (= seq_lens) */
    int page_size, n_pages, max_pages, max_seq_len;
    const float* rope_table;      /* anelm_rope_table rows, or NULL */
    int rope_rows;
    /* optional LM head: top_k of lm_w rmsnorm(x[b], final_norm_w) */
    const float* final_norm_w;    /* NULL: x as is */
    const uint8_t* lm_w;          /* NULL: no LM head */
    const uint16_t* lm_lut;
    int vocab, top_k;
    int32_t* top_idx;             /* [B][top_k] */
    float* top_val;
} anelm_batch_seqs;

typedef struct anelm_batch_step anelm_batch_step;

/* Copies the descriptors; allocates the step's activation scratch. */
int anelm_batch_step_create(anelm_batch_step** out, const anelm_hybrid_dims* dims,
                            const anelm_batch_layer* layers, int n_layers,
                            const anelm_batch_seqs* seqs, float* x);
/* One step for every sequence; with `advance`, seq_lens (and positions) are
 * incremented on the device afterwards, as the KV caches grew by one key.  A
 * sequence whose cache already held max_seq_len keys appended nothing: it is
 * not advanced, and the step's status records it. */
int anelm_batch_step_run(anelm_batch_step* step, int advance, void* stream);
/* Synchronous: *status = 1 if, since the last call, an advancing run found a
 * sequence at max_seq_len keys (its new key was not cached), else 0; clears
 * the flag.  No counterpart in the reference (its ring caches slide,
 * qwen3_5.cpp:973-983; a paged cache of fixed size cannot). */
int anelm_batch_step_status(anelm_batch_step* step, int* status);
int anelm_batch_step_destroy(anelm_batch_step* step);

#ifdef __cplusplus
}
#endif
#endif /* ANELM_H */
