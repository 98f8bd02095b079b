// Batched decode step executor: the layer loop of Qwen35Model::forward
// (models/llm/qwen3_5.cpp:1278-1356) over the compute cores for a batch of
// concurrent sequences, each with its own paged fp16 KV cache and DeltaNet
// state (the reference serves one request at a time, main.cpp:276-371; here
// one step advances every sequence by one token).  Per layer:
//   full attention  anelm_attn_decode_paged_step (norms, RoPE, page append,
//                   attention, gate per sequence), or
//   DeltaNet        one launch over all sequences' value heads;
//   FFN             x[b] += down(silu(gate n_b) * (up n_b)),
//                   n_b = rmsnorm(x[b], ffn_norm_w) -- gate and up as one
//                   stacked projection, each weight dequantised once per 32
//                   sequences (anelm_lut6_gemm).
// Optionally the final norm and the LM-head top-k.  Scratch activations are
// owned by the step (allocated at create).
#include "anelm_internal.hpp"

#include <vector>

struct anelm_batch_step {
    anelm_hybrid_dims dims;
    anelm_batch_seqs seqs;
    std::vector<anelm_batch_layer> layers;
    float* x = nullptr;        // [B][H], caller's
    float* xn = nullptr;       // [B][H]
    float* gu = nullptr;       // [B][2I]
    float* h = nullptr;        // [B][I]
    int32_t* status = nullptr; // device word: a sequence reached max_seq_len
};

namespace anelm {
namespace {

// A sequence whose cache held max_seq_len keys before the step appended
// nothing (anelm_attn_decode_paged_step): it does not advance, and the step's
// status word records that it hit the limit.
__global__ void advance_kernel(int32_t* seq_lens, int32_t* positions, int n, int max_seq_len, int32_t* status) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        if (seq_lens[i] >= max_seq_len) {
            *status = 1;
            return;
        }
        seq_lens[i] += 1;
        if (positions) positions[i] += 1;
    }
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_batch_step_create(anelm_batch_step** out, const anelm_hybrid_dims* dims,
                                       const anelm_batch_layer* layers, int n_layers,
                                       const anelm_batch_seqs* seqs, float* x) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(dims);
    ANELM_NONNULL(layers);
    ANELM_NONNULL(seqs);
    ANELM_NONNULL(x);
    ANELM_NONNULL(seqs->seq_lens);
    *out = nullptr;
    ANELM_REQUIRE(n_layers > 0, "batch_step: n_layers %d", n_layers);
    ANELM_REQUIRE(seqs->n_seqs > 0 && seqs->n_seqs <= 1024, "batch_step: n_seqs %d (1..1024)", seqs->n_seqs);
    ANELM_REQUIRE(dims->hidden > 0 && dims->inter > 0, "batch_step: hidden %d inter %d", dims->hidden, dims->inter);
    for (int i = 0; i < n_layers; i++) {
        const anelm_batch_layer& L = layers[i];
        ANELM_REQUIRE(L.kind == ANELM_LAYER_ATTENTION || L.kind == ANELM_LAYER_DELTANET,
                      "batch_step: layer %d kind %d", i, L.kind);
        ANELM_REQUIRE(L.core_out && L.ffn_norm_w && L.gate_up_w && L.gate_up_lut && L.down_w && L.down_lut,
                      "batch_step: layer %d misses its output or FFN weights", i);
        if (L.kind == ANELM_LAYER_ATTENTION)
            ANELM_REQUIRE(L.q_gate && L.k && L.v && L.k_pages && L.v_pages && L.page_table,
                          "batch_step: attention layer %d misses inputs or pages", i);
        else
            ANELM_REQUIRE(L.state && L.dn_q && L.dn_k && L.dn_v && L.dn_a && L.dn_b && L.dn_A && L.dn_dt_bias,
                          "batch_step: DeltaNet layer %d misses inputs", i);
    }
    if (seqs->lm_w) {
        ANELM_REQUIRE(seqs->lm_lut && seqs->top_idx && seqs->top_val && seqs->vocab > 0 && seqs->top_k > 0,
                      "batch_step: LM head needs lut, outputs, vocab and top_k");
    }
    auto* s = new anelm_batch_step();
    s->dims = *dims;
    s->seqs = *seqs;
    s->layers.assign(layers, layers + n_layers);
    s->x = x;
    const size_t B = (size_t)seqs->n_seqs, H = dims->hidden, I = dims->inter;
    hipError_t e = hipMalloc(&s->xn, B * H * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&s->gu, B * 2 * I * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&s->h, B * I * sizeof(float));
    if (e == hipSuccess) e = hipMalloc(&s->status, sizeof(int32_t));
    if (e == hipSuccess) e = hipMemset(s->status, 0, sizeof(int32_t));
    if (e != hipSuccess) {
        anelm_batch_step_destroy(s);
        return hip_fail(e, "hipMalloc(batch step scratch)");
    }
    *out = s;
    return ANELM_OK;
}

extern "C" int anelm_batch_step_run(anelm_batch_step* s, int advance, void* stream) {
    ANELM_NONNULL(s);
    const anelm_hybrid_dims& d = s->dims;
    const anelm_batch_seqs& q = s->seqs;
    const int B = q.n_seqs, H = d.hidden, I = d.inter;
    const int n_layers = (int)s->layers.size();
    // the final norm for the LM head, folded into the last down projection
    const float* final_norm = q.lm_w ? q.final_norm_w : nullptr;
    for (int l = 0; l < n_layers; l++) {
        const anelm_batch_layer& L = s->layers[l];
        int rc;
        if (L.kind == ANELM_LAYER_ATTENTION) {
            rc = anelm_attn_decode_paged_step(L.core_out, L.q_gate, L.k, L.v, L.k_pages, L.v_pages, L.page_table,
                                              q.seq_lens, q.positions, L.q_norm_w, L.k_norm_w, q.rope_table,
                                              q.rope_rows, B, q.max_pages, q.page_size, q.n_pages, q.max_seq_len,
                                              d.n_heads, d.n_kv_heads, d.head_dim, d.rot_dim, d.theta, d.eps,
                                              d.rope_mode, 1, stream);
        } else {
            rc = anelm_deltanet_decode_batched(L.core_out, L.state, L.dn_q, L.dn_k, L.dn_v, L.dn_a, L.dn_b, L.dn_A,
                                               L.dn_dt_bias, L.dn_z, L.dn_norm_w, B, d.lin_k_heads, d.lin_v_heads,
                                               d.lin_dim, d.lin_dim, L.dn_flags, stream);
        }
        if (rc) return rc;
        // the FFN norm of layer 0; later layers' come with the previous down
        // projection (the cores between leave x unchanged)
        if (l == 0) {
            rc = anelm_rmsnorm(s->xn, s->x, L.ffn_norm_w, H, B, H, H, d.eps, stream);
            if (rc) return rc;
        }
        rc = anelm_lut6_gemm(s->gu, L.gate_up_w, L.gate_up_lut, s->xn, B, 2 * I, H, 0, stream);
        if (rc) return rc;
        rc = anelm_swiglu_rows(s->h, s->gu, B, I, stream);
        if (rc) return rc;
        const float* next_norm = l + 1 < n_layers ? s->layers[l + 1].ffn_norm_w : final_norm;
        rc = next_norm ? lut6_gemm_norm(s->x, L.down_w, L.down_lut, s->h, B, H, I, 1, next_norm, d.eps, s->xn,
                                        as_stream(stream))
                       : anelm_lut6_gemm(s->x, L.down_w, L.down_lut, s->h, B, H, I, 1, stream);
        if (rc) return rc;
    }
    if (q.lm_w) {
        const float* xf = final_norm ? s->xn : s->x;
        if (final_norm && n_layers == 0) {
            const int rc = anelm_rmsnorm(s->xn, s->x, final_norm, H, B, H, H, d.eps, stream);
            if (rc) return rc;
        }
        const int rc = anelm_lut6_topk(q.top_idx, q.top_val, q.lm_w, q.lm_lut, xf, B, q.vocab, H, q.top_k, stream);
        if (rc) return rc;
    }
    if (advance) {
        hipLaunchKernelGGL(advance_kernel, dim3((B + 255) / 256), dim3(256), 0, as_stream(stream), q.seq_lens,
                           q.positions, B, q.max_seq_len, s->status);
        ANELM_LAUNCHED("advance_kernel");
    }
    return ANELM_OK;
}

extern "C" int anelm_batch_step_status(anelm_batch_step* s, int* status) {
    ANELM_NONNULL(s);
    ANELM_NONNULL(status);
    int32_t v = 0;
    ANELM_HIP(hipMemcpy(&v, s->status, sizeof(v), hipMemcpyDeviceToHost));
    *status = v;
    if (v) ANELM_HIP(hipMemset(s->status, 0, sizeof(int32_t)));
    return ANELM_OK;
}

extern "C" int anelm_batch_step_destroy(anelm_batch_step* s) {
    if (!s) return ANELM_OK;
    if (s->status) (void)hipFree(s->status);
    if (s->xn) (void)hipFree(s->xn);
    if (s->gu) (void)hipFree(s->gu);
    if (s->h) (void)hipFree(s->h);
    delete s;
    return ANELM_OK;
}
