/*
 * anelm_cpu_ops.h -- link-time drop-in for the reference's core/cpu_ops.h.
 *
 * Same namespace (ane_lm), names, argument order and meaning as
 * core/cpu_ops.h:12-58; buffers are caller-owned HOST fp32 arrays and every
 * call is synchronous, exactly like the reference.  Each function stages its
 * operands to the current HIP device, runs the libanelm kernel and copies the
 * results back -- a correctness path for existing callers (generate.cpp,
 * qwen3_5.cpp, sampling.cpp); the native tier in anelm.h keeps data resident.
 *
 * The reference functions return void and cannot fail; here a failing call
 * (bad shape, no device) prints anelm_last_error() and aborts rather than
 * returning silently wrong results.
 */
#ifndef ANELM_CPU_OPS_H
#define ANELM_CPU_OPS_H

#include <math.h>
#include <stdio.h>
#include <stdlib.h>

#include "anelm.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Host-pointer, synchronous forms; 0 = ok, < 0 = anelm error code. */
int anelm_cpu_silu_vec_inplace(float* x, int n, float* tmp);
int anelm_cpu_mul_sigmoid_inplace(float* y, const float* z, int n, float* tmp);
int anelm_cpu_rmsnorm(float* out, const float* x, const float* weight, int dim, float eps);
int anelm_cpu_rmsnorm_gated(float* out, const float* x, const float* z, const float* weight, int dim);
int anelm_cpu_apply_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                                int q_head_stride, int k_head_stride, int rot_dim, int pos,
                                float theta, const float* cos_row, const float* sin_row);
int anelm_cpu_softmax(float* x, int n);
int anelm_cpu_matvec(float* y, const float* W, const float* x, int out_dim, int in_dim);
int anelm_cpu_l2_normalize(float* x, int dim);
int anelm_cpu_conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                            const float* w, int channels, int kernel_size);
int anelm_cpu_ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                       float decay, float beta, int key_dim, int value_dim);
int anelm_cpu_gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                            int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                            int cache_start, int cache_len, int cache_capacity);

#ifdef __cplusplus
}  /* extern "C" */

namespace ane_lm {

inline void anelm_check_(int rc, const char* fn) {
    if (rc != 0) {
        fprintf(stderr, "ane_lm::%s (libanelm) failed: %s\n", fn, anelm_last_error());
        abort();
    }
}

/* core/cpu_ops.h:12-14 */
inline float silu_f(float x) { return x / (1.0f + expf(-x)); }
inline float sigmoid_f(float x) { return 1.0f / (1.0f + expf(-x)); }
inline float softplus_f(float x) { return logf(1.0f + expf(x)); }

/* core/cpu_ops.h:16-17 */
inline void silu_vec_inplace(float* x, int n, float* tmp) {
    anelm_check_(anelm_cpu_silu_vec_inplace(x, n, tmp), "silu_vec_inplace");
}
inline void mul_sigmoid_inplace(float* y, const float* z, int n, float* tmp) {
    anelm_check_(anelm_cpu_mul_sigmoid_inplace(y, z, n, tmp), "mul_sigmoid_inplace");
}
/* core/cpu_ops.h:21-22 */
inline void rmsnorm(float* out, const float* x, const float* weight, int dim, float eps = 1e-6f) {
    anelm_check_(anelm_cpu_rmsnorm(out, x, weight, dim, eps), "rmsnorm");
}
inline void rmsnorm_gated(float* out, const float* x, const float* z, const float* weight, int dim) {
    anelm_check_(anelm_cpu_rmsnorm_gated(out, x, z, weight, dim), "rmsnorm_gated");
}
/* core/cpu_ops.h:26-29 */
inline void apply_rope_cached(float* q, float* k, int n_q_heads, int n_kv_heads, int head_dim,
                              int q_head_stride, int k_head_stride, int rot_dim, int pos,
                              float theta, const float* cos_row, const float* sin_row) {
    anelm_check_(anelm_cpu_apply_rope_cached(q, k, n_q_heads, n_kv_heads, head_dim, q_head_stride,
                                             k_head_stride, rot_dim, pos, theta, cos_row, sin_row),
                 "apply_rope_cached");
}
/* core/cpu_ops.h:33-41 */
inline void softmax(float* x, int n) { anelm_check_(anelm_cpu_softmax(x, n), "softmax"); }
inline void matvec(float* y, const float* W, const float* x, int out_dim, int in_dim) {
    anelm_check_(anelm_cpu_matvec(y, W, x, out_dim, in_dim), "matvec");
}
inline void l2_normalize(float* x, int dim) {
    anelm_check_(anelm_cpu_l2_normalize(x, dim), "l2_normalize");
}
/* core/cpu_ops.h:45-46 */
inline void conv1d_update(float* y, float* conv_state, int* state_pos, const float* x,
                          const float* w, int channels, int kernel_size) {
    anelm_check_(anelm_cpu_conv1d_update(y, conv_state, state_pos, x, w, channels, kernel_size),
                 "conv1d_update");
}
/* core/cpu_ops.h:50-51 */
inline void ssm_step(float* y, float* state, const float* q, const float* k, const float* v,
                     float decay, float beta, int key_dim, int value_dim) {
    anelm_check_(anelm_cpu_ssm_step(y, state, q, k, v, decay, beta, key_dim, value_dim), "ssm_step");
}
/* core/cpu_ops.h:55-58 */
inline void gqa_attention(float* out, const float* q, const float* k_cache, const float* v_cache,
                          int n_heads, int n_kv_heads, int head_dim, int q_head_stride,
                          int cache_start, int cache_len, int cache_capacity) {
    anelm_check_(anelm_cpu_gqa_attention(out, q, k_cache, v_cache, n_heads, n_kv_heads, head_dim,
                                         q_head_stride, cache_start, cache_len, cache_capacity),
                 "gqa_attention");
}

}  // namespace ane_lm
#endif /* __cplusplus */

#endif /* ANELM_CPU_OPS_H */
