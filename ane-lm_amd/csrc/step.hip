// Hybrid decode step executor: the per-layer core + FFN launch sequence of
// Qwen35Model::forward (models/llm/qwen3_5.cpp:1278-1356), issued from C++ and
// optionally captured once into a HIP graph so a step costs one graph launch
// instead of ~3 host launches per layer.
#include "anelm_internal.hpp"

#include <vector>

struct anelm_hybrid_step {
    anelm_hybrid_dims dims;
    std::vector<anelm_hybrid_layer> layers;
    float* x = nullptr;
    float* h = nullptr;
    bool use_graph = false;
    int mode = 0;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    anelm::PersistentStep* ps = nullptr;
    // split partials of the attention layers (graph mode): owned by the step,
    // so the captured launches never point into the shared workspace, which a
    // later call may free when it grows
    float* part = nullptr;
    size_t part_bytes = 0;
};

namespace anelm {
namespace {

// Rows of a layer's first projection: attention q_gate | k | v
// (qwen3_5.cpp:948-950), DeltaNet mixed qkv | z | a | b (:849-860).
int first_out(const anelm_hybrid_dims& d, bool attn) {
    if (attn) return d.n_heads * 2 * d.head_dim + 2 * d.n_kv_heads * d.head_dim;
    return 2 * d.lin_k_heads * d.lin_dim + 2 * d.lin_v_heads * d.lin_dim + 2 * d.lin_v_heads;
}

// One eager pass over all layers; `advance` moves every attention ring one
// token forward (the host-side KVCache bookkeeping of qwen3_5.cpp:973-983).
int launch_all(anelm_hybrid_step* s, hipStream_t st, bool advance) {
    const anelm_hybrid_dims& d = s->dims;
    for (auto& L : s->layers) {
        int rc;
        const bool proj = L.first_w != nullptr;
        const bool attn = L.kind == ANELM_LAYER_ATTENTION;
        if (proj) {
            // proj = first_w rmsnorm(x, in_norm_w) (qwen3_5.cpp:1287-1300, 1004-1011)
            rc = lut6_gemv_impl(L.proj, L.first_w, L.first_lut, s->x, L.in_norm_w, d.eps, first_out(d, attn),
                                d.hidden, 0, st);
            if (rc) return rc;
        }
        if (attn) {
            int start = L.cache_start, len = L.cache_len;
            const float* q_gate = proj ? L.proj : L.q_gate;
            const float* k = proj ? L.proj + (size_t)d.n_heads * 2 * d.head_dim : L.k;
            const float* v = proj ? k + (size_t)d.n_kv_heads * d.head_dim : L.v;
            rc = full_attn_decode_impl(L.core_out, q_gate, k, v, L.k_cache, L.v_cache, L.q_norm_w,
                                       L.k_norm_w, d.n_heads, d.n_kv_heads, d.head_dim, d.rot_dim, L.pos,
                                       d.theta, d.eps, d.rope_mode, 1, nullptr, nullptr, &start, &len,
                                       L.cache_capacity, st, s->part, s->part_bytes);
            if (rc) return rc;
            if (advance) {
                L.cache_start = start;
                L.cache_len = len;
                L.pos++;
            }
        } else if (proj) {
            // conv ring + SiLU + split + recurrence from the projection (:849-908)
            int pos = L.conv_pos;
            rc = anelm_deltanet_decode_from_proj(L.core_out, L.state, L.conv_state, &pos, L.proj, L.conv_w,
                                                 L.dn_A, L.dn_dt_bias, L.dn_norm_w, d.lin_k_heads, d.lin_v_heads,
                                                 d.lin_dim, d.lin_dim, d.conv_kernel, L.dn_flags, st);
            if (rc) return rc;
            if (advance) L.conv_pos = pos;
        } else {
            rc = anelm_deltanet_decode(L.core_out, L.state, L.dn_q, L.dn_k, L.dn_v, L.dn_a, L.dn_b,
                                       L.dn_A, L.dn_dt_bias, L.dn_z, L.dn_norm_w, d.lin_k_heads,
                                       d.lin_v_heads, d.lin_dim, d.lin_dim, L.dn_flags, st);
            if (rc) return rc;
        }
        if (proj) {
            // x += o_proj(core_out) (:1310-1327)
            const int attn_dim = attn ? d.n_heads * d.head_dim : d.lin_v_heads * d.lin_dim;
            rc = lut6_gemv_impl(s->x, L.o_w, L.o_lut, L.core_out, nullptr, 0.f, d.hidden, attn_dim, 1, st);
            if (rc) return rc;
        }
        rc = anelm_lut6_ffn(s->x, s->h, L.ffn_norm_w, d.eps, L.gate_w, L.gate_lut, L.up_w, L.up_lut,
                            L.down_w, L.down_lut, d.hidden, d.inter, st);
        if (rc) return rc;
    }
    return ANELM_OK;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_hybrid_step_create(anelm_hybrid_step** out, const anelm_hybrid_dims* dims,
                                        const anelm_hybrid_layer* layers, int n_layers, float* x,
                                        float* h_scratch, int mode, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(dims);
    ANELM_NONNULL(layers);
    ANELM_NONNULL(x);
    ANELM_NONNULL(h_scratch);
    ANELM_REQUIRE(n_layers > 0, "hybrid_step: n_layers %d", n_layers);
    ANELM_REQUIRE(mode == ANELM_STEP_EAGER || mode == ANELM_STEP_GRAPH ||
                      ((mode & ANELM_STEP_PERSISTENT) &&
                       (mode & ~(ANELM_STEP_PERSISTENT | ANELM_STEP_STATIC | ANELM_STEP_COOPERATIVE)) == 0),
                  "hybrid_step: mode %d unknown", mode);
    const bool use_graph = mode == ANELM_STEP_GRAPH;
    ANELM_REQUIRE(!use_graph || stream != nullptr, "hybrid_step: graph capture needs a non-null stream");
    for (int i = 0; i < n_layers; i++) {
        const anelm_hybrid_layer& L = layers[i];
        ANELM_REQUIRE(L.kind == ANELM_LAYER_ATTENTION || L.kind == ANELM_LAYER_DELTANET,
                      "hybrid_step: layer %d kind %d", i, L.kind);
        if (!L.first_w) continue;
        ANELM_REQUIRE(L.first_lut && L.o_w && L.o_lut && L.proj,
                      "hybrid_step: layer %d has a first projection but no o_proj / proj scratch", i);
        ANELM_REQUIRE(L.kind == ANELM_LAYER_ATTENTION ||
                          (L.conv_state && L.conv_w && dims->conv_kernel >= 2 && L.conv_pos >= 0 &&
                           L.conv_pos < dims->conv_kernel - 1),
                      "hybrid_step: DeltaNet layer %d needs the conv ring (kernel %d, pos %d)", i,
                      dims->conv_kernel, L.conv_pos);
    }
    auto* s = new anelm_hybrid_step();
    s->dims = *dims;
    s->layers.assign(layers, layers + n_layers);
    s->x = x;
    s->h = h_scratch;
    s->use_graph = use_graph;
    s->mode = mode;
    hipStream_t st = as_stream(stream);
    if (mode & ANELM_STEP_PERSISTENT) {
        const int rc = persistent_create(&s->ps, dims, layers, n_layers, x, h_scratch, st);
        if (rc != ANELM_OK) {
            delete s;
            return rc;
        }
        *out = s;
        return ANELM_OK;
    }
    if (s->use_graph) {
        // The captured launches allocate nothing: the attention layers' split
        // partials go to a buffer of the step, sized for full rings; the FFN
        // blocks use h_scratch.  No step runs before the capture.
        // the capture stream's counters and workspace exist before the
        // capture (their creation launches a fill kernel and allocates)
        int rc = stream_state(st) ? ANELM_OK : ANELM_EHIP;
        for (int i = 0; i < n_layers && rc == ANELM_OK; i++)
            if (layers[i].kind == ANELM_LAYER_ATTENTION) {
                const size_t need = full_attn_part_bytes(dims->n_heads, dims->n_kv_heads, dims->head_dim,
                                                         layers[i].cache_capacity);
                if (need > s->part_bytes) s->part_bytes = need;
            }
        if (rc == ANELM_OK && s->part_bytes > 0) {
            hipError_t e = hipMalloc(&s->part, s->part_bytes);
            if (e != hipSuccess) rc = hip_fail(e, "hipMalloc(step partials)");
            // the arrival counters at its end start at zero (the launches
            // leave them zero)
            if (rc == ANELM_OK) {
                e = hipMemset(s->part, 0, s->part_bytes);
                if (e == hipSuccess) e = hipDeviceSynchronize();
                if (e != hipSuccess) rc = hip_fail(e, "hipMemset(step partials)");
            }
        }
        if (rc == ANELM_OK) {
            hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
            if (e != hipSuccess) rc = hip_fail(e, "hipStreamBeginCapture");
            else {
                rc = launch_all(s, st, false);
                hipGraph_t g = nullptr;
                e = hipStreamEndCapture(st, &g);
                if (rc == ANELM_OK && e != hipSuccess) rc = hip_fail(e, "hipStreamEndCapture");
                s->graph = g;
                if (rc == ANELM_OK) {
                    e = hipGraphInstantiate(&s->exec, g, nullptr, nullptr, 0);
                    if (e != hipSuccess) rc = hip_fail(e, "hipGraphInstantiate");
                }
            }
        }
        if (rc != ANELM_OK) {
            anelm_hybrid_step_destroy(s);
            return rc;
        }
    }
    *out = s;
    return ANELM_OK;
}

extern "C" int anelm_hybrid_step_run(anelm_hybrid_step* step, void* stream) {
    ANELM_NONNULL(step);
    hipStream_t st = as_stream(stream);
    if (step->ps)
        return persistent_run(step->ps, (step->mode & ANELM_STEP_STATIC) == 0,
                              (step->mode & ANELM_STEP_COOPERATIVE) != 0, st);
    if (step->use_graph) {
        ANELM_HIP(hipGraphLaunch(step->exec, st));
        return ANELM_OK;
    }
    return launch_all(step, st, true);
}

extern "C" int anelm_hybrid_step_status(anelm_hybrid_step* step, int* status) {
    ANELM_NONNULL(step);
    ANELM_NONNULL(status);
    *status = 0;
    return step->ps ? persistent_status(step->ps, status) : ANELM_OK;
}

extern "C" int anelm_hybrid_step_trace(anelm_hybrid_step* step, uint64_t* host, size_t n_words, int* grid,
                                       int* phases) {
    ANELM_NONNULL(step);
    ANELM_NONNULL(host);
    ANELM_NONNULL(grid);
    ANELM_NONNULL(phases);
    ANELM_REQUIRE(step->ps != nullptr, "step trace: only the persistent step records a timeline");
    return persistent_trace(step->ps, reinterpret_cast<unsigned long long*>(host), n_words, grid, phases);
}

extern "C" int anelm_hybrid_step_destroy(anelm_hybrid_step* step) {
    if (!step) return ANELM_OK;
    if (step->ps) persistent_destroy(step->ps);
    if (step->exec) (void)hipGraphExecDestroy(step->exec);
    if (step->graph) (void)hipGraphDestroy(step->graph);
    if (step->part) (void)hipFree(step->part);
    delete step;
    return ANELM_OK;
}
