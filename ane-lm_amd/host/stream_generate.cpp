// stream_generate over the libanelm C ABI: the decode loop of
// generate.cpp:30-140 (stream_generate) for a Qwen3.5-shaped hybrid model
// whose whole forward runs on the GPU.
//
//   prefill: one forward per prompt token (the single-token path,
//            generate.cpp:76-84), the LM head only after the last; or
//            (PREFILL_MODE 1) the whole prompt through each layer at once,
//            as Qwen35Model::forward_batch (models/llm/qwen3_5.cpp:1164-1217)
//            batches the projections -- here the cores take the prompt in
//            one call too (anelm_full_attn_prefill,
//            anelm_deltanet_prefill_from_proj);
//   decode:  sample_token over the logits with the generated tokens as the
//            penalty window (generate.cpp:96-104, core/sampling.cpp:11-66),
//            then forward(next token) until max_tokens.
//
// forward(token, pos) is Qwen35Model::forward (models/llm/qwen3_5.cpp:
// 1278-1417): the embedding row, ONE anelm_hybrid_step run over the
// complete layers (projections, conv ring / DeltaNet or attention core,
// o_proj, FFN), the final norm and the LUT6 LM head.
//
// Usage: stream_generate MODEL PROMPT MAX_TOKENS TEMPERATURE REP_PENALTY
//                        REP_CONTEXT FREQ_PENALTY SEED [PREFILL_MODE]
//   MODEL   weights as written by tests/test_gpu_host_loop.py: a sequence
//           of records (int64 byte count, bytes) in a fixed order;
//   PROMPT  comma-separated token ids.
// Prints "token <id>" per generated token, then "done <n> <tokens/s>".
// The uniform draws come from a seeded 64-bit LCG (the reference uses
// drand48(), core/sampling.cpp:57).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/anelm.h"

namespace {

#define CHECK(call)                                                                        \
    do {                                                                                   \
        int rc_ = (call);                                                                  \
        if (rc_ != 0) {                                                                    \
            fprintf(stderr, "%s failed (%d): %s\n", #call, rc_, anelm_last_error());     \
            exit(1);                                                                       \
        }                                                                                  \
    } while (0)
#define HIPCHECK(call)                                                                     \
    do {                                                                                   \
        hipError_t e_ = (call);                                                            \
        if (e_ != hipSuccess) {                                                            \
            fprintf(stderr, "%s failed: %s\n", #call, hipGetErrorString(e_));              \
            exit(1);                                                                       \
        }                                                                                  \
    } while (0)

struct Reader {
    FILE* f;
    std::vector<char> next() {
        int64_t n = 0;
        if (fread(&n, sizeof(n), 1, f) != 1 || n < 0) {
            fprintf(stderr, "model file truncated\n");
            exit(1);
        }
        std::vector<char> b((size_t)n);
        if (n && fread(b.data(), 1, (size_t)n, f) != (size_t)n) {
            fprintf(stderr, "model file truncated\n");
            exit(1);
        }
        return b;
    }
};

std::vector<void*> g_allocs;

void* upload(const std::vector<char>& b) {
    void* d = nullptr;
    HIPCHECK(hipMalloc(&d, b.size() ? b.size() : 4));
    if (!b.empty()) HIPCHECK(hipMemcpy(d, b.data(), b.size(), hipMemcpyHostToDevice));
    g_allocs.push_back(d);
    return d;
}

void* zeros(size_t bytes) {
    void* d = nullptr;
    HIPCHECK(hipMalloc(&d, bytes));
    HIPCHECK(hipMemset(d, 0, bytes));
    g_allocs.push_back(d);
    return d;
}

struct Model {
    int hidden, inter, n_layers, n_heads, n_kv_heads, head_dim, rot_dim, lin_k, lin_v, lin_dim, conv_k,
        vocab, cap, max_first;
    float theta, eps;
    std::vector<anelm_hybrid_layer> layers;
    float* embed;
    float* final_norm;
    uint8_t* lm_w;
    uint16_t* lm_lut;
};

Model load(const char* path) {
    Model m{};
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "cannot open %s\n", path);
        exit(1);
    }
    Reader r{f};
    std::vector<char> hdr = r.next();
    const int32_t* h = reinterpret_cast<const int32_t*>(hdr.data());
    if (hdr.size() != 15 * 4) {
        fprintf(stderr, "bad header\n");
        exit(1);
    }
    m.hidden = h[0], m.inter = h[1], m.n_layers = h[2], m.n_heads = h[3], m.n_kv_heads = h[4], m.head_dim = h[5];
    m.rot_dim = h[6], m.lin_k = h[7], m.lin_v = h[8], m.lin_dim = h[9], m.conv_k = h[10], m.vocab = h[11];
    m.cap = h[12];
    memcpy(&m.theta, &h[13], 4);
    memcpy(&m.eps, &h[14], 4);
    const int qkv = 2 * m.lin_k * m.lin_dim + m.lin_v * m.lin_dim;
    for (int i = 0; i < m.n_layers; i++) {
        anelm_hybrid_layer L;
        memset(&L, 0, sizeof(L));
        L.kind = (i + 1) % 4 == 0 ? ANELM_LAYER_ATTENTION : ANELM_LAYER_DELTANET;   // qwen3_5.cpp:64-71
        L.in_norm_w = static_cast<float*>(upload(r.next()));
        std::vector<char> fw = r.next();
        const int first_out = (int)(fw.size() * 4 / 3 / m.hidden);
        if (first_out > m.max_first) m.max_first = first_out;
        L.first_w = static_cast<uint8_t*>(upload(fw));
        L.first_lut = static_cast<uint16_t*>(upload(r.next()));
        L.o_w = static_cast<uint8_t*>(upload(r.next()));
        L.o_lut = static_cast<uint16_t*>(upload(r.next()));
        L.ffn_norm_w = static_cast<float*>(upload(r.next()));
        L.gate_w = static_cast<uint8_t*>(upload(r.next()));
        L.gate_lut = static_cast<uint16_t*>(upload(r.next()));
        L.up_w = static_cast<uint8_t*>(upload(r.next()));
        L.up_lut = static_cast<uint16_t*>(upload(r.next()));
        L.down_w = static_cast<uint8_t*>(upload(r.next()));
        L.down_lut = static_cast<uint16_t*>(upload(r.next()));
        L.proj = static_cast<float*>(zeros((size_t)first_out * 4));
        if (L.kind == ANELM_LAYER_ATTENTION) {
            L.q_norm_w = static_cast<float*>(upload(r.next()));
            L.k_norm_w = static_cast<float*>(upload(r.next()));
            const size_t kv = (size_t)m.cap * m.n_kv_heads * m.head_dim * 2;
            L.k_cache = static_cast<uint16_t*>(zeros(kv));
            L.v_cache = static_cast<uint16_t*>(zeros(kv));
            L.cache_capacity = m.cap;
            L.core_out = static_cast<float*>(zeros((size_t)m.n_heads * m.head_dim * 4));
        } else {
            L.conv_w = static_cast<float*>(upload(r.next()));
            L.dn_A = static_cast<float*>(upload(r.next()));
            L.dn_dt_bias = static_cast<float*>(upload(r.next()));
            L.dn_norm_w = static_cast<float*>(upload(r.next()));
            L.state = static_cast<float*>(zeros((size_t)m.lin_v * m.lin_dim * m.lin_dim * 4));
            L.conv_state = static_cast<float*>(zeros((size_t)qkv * (m.conv_k - 1) * 4));
            L.dn_flags = ANELM_DN_L2NORM | ANELM_DN_GATED_NORM;
            L.core_out = static_cast<float*>(zeros((size_t)m.lin_v * m.lin_dim * 4));
        }
        m.layers.push_back(L);
    }
    m.embed = static_cast<float*>(upload(r.next()));
    m.final_norm = static_cast<float*>(upload(r.next()));
    m.lm_w = static_cast<uint8_t*>(upload(r.next()));
    m.lm_lut = static_cast<uint16_t*>(upload(r.next()));
    fclose(f);
    return m;
}

struct Lcg {
    uint64_t s;
    double next() {   // uniform in [0, 1) from the top 53 bits
        s = s * 6364136223846793005ull + 1442695040888963407ull;
        return (double)(s >> 11) * (1.0 / 9007199254740992.0);
    }
};

}  // namespace

int main(int argc, char** argv) {
    if (argc != 9 && argc != 10) {
        fprintf(stderr,
                "usage: %s MODEL PROMPT MAX_TOKENS TEMPERATURE REP_PENALTY REP_CONTEXT FREQ_PENALTY SEED "
                "[PREFILL_MODE]\n",
                argv[0]);
        return 2;
    }
    const int prefill_mode = argc == 10 ? atoi(argv[9]) : 0;
    Model m = load(argv[1]);
    std::vector<int> prompt;
    for (const char* p = argv[2]; *p;) {
        prompt.push_back((int)strtol(p, const_cast<char**>(&p), 10));
        if (*p == ',') p++;
    }
    const int max_tokens = atoi(argv[3]);
    const float temperature = (float)atof(argv[4]), rep = (float)atof(argv[5]), freq = (float)atof(argv[7]);
    const int rep_ctx = atoi(argv[6]);
    Lcg rng{strtoull(argv[8], nullptr, 10)};
    if (prompt.empty() || max_tokens < 0 || (int)prompt.size() + max_tokens > m.cap) {
        fprintf(stderr, "prompt + max_tokens must fit the %d-slot caches\n", m.cap);
        return 2;
    }

    hipStream_t st;
    HIPCHECK(hipStreamCreate(&st));
    float* x = static_cast<float*>(zeros((size_t)m.hidden * 4));
    float* xf = static_cast<float*>(zeros((size_t)m.hidden * 4));
    float* h = static_cast<float*>(zeros((size_t)m.inter * 2 * 4));
    float* logits = static_cast<float*>(zeros((size_t)m.vocab * 4));
    int32_t* d_token = static_cast<int32_t*>(zeros(4));
    int32_t* d_recent = static_cast<int32_t*>(zeros((size_t)(max_tokens + 1) * 4));
    anelm_hybrid_dims dims{m.hidden, m.inter, m.n_heads, m.n_kv_heads, m.head_dim, m.rot_dim,
                           ANELM_ROPE_INTERLEAVED, m.theta, m.eps, m.lin_k, m.lin_v, m.lin_dim, m.conv_k};
    anelm_hybrid_step* step = nullptr;

    // Qwen35Model::forward(token, pos, compute_logits)
    auto forward = [&](int token, bool compute_logits) {
        HIPCHECK(hipMemcpyAsync(x, m.embed + (size_t)token * m.hidden, (size_t)m.hidden * 4,
                                hipMemcpyDeviceToDevice, st));
        CHECK(anelm_hybrid_step_run(step, st));
        if (!compute_logits) return;
        CHECK(anelm_rmsnorm(xf, x, m.final_norm, m.hidden, 1, m.hidden, m.hidden, m.eps, st));
        CHECK(anelm_lut6_gemv(logits, m.lm_w, m.lm_lut, xf, m.vocab, m.hidden, st));
    };

    // Qwen35Model::forward_batch(tokens, S, 0) over the whole prompt, then the
    // LM head on its last row.  Per layer: input norm and the first projection
    // for all tokens, the core over the prompt, o_proj + residual, the FFN
    // block; the rings and conv state end as after S single-token forwards.
    auto prefill_batch = [&](const std::vector<int>& toks) {
        const int S = (int)toks.size(), H = m.hidden, I = m.inter;
        const int core_max = std::max(m.n_heads * m.head_dim, m.lin_v * m.lin_dim);
        float* X = static_cast<float*>(zeros((size_t)S * H * 4));
        float* XN = static_cast<float*>(zeros((size_t)S * H * 4));
        float* P = static_cast<float*>(zeros((size_t)S * m.max_first * 4));
        float* C = static_cast<float*>(zeros((size_t)S * core_max * 4));
        float* G = static_cast<float*>(zeros((size_t)S * I * 4));
        float* U = static_cast<float*>(zeros((size_t)S * I * 4));
        float* rope = static_cast<float*>(zeros((size_t)m.cap * m.rot_dim * 4));
        CHECK(anelm_rope_table(rope, m.rot_dim, m.cap, m.theta));   // qwen3_5.cpp:308-324
        for (int t = 0; t < S; t++)
            HIPCHECK(hipMemcpyAsync(X + (size_t)t * H, m.embed + (size_t)toks[t] * H, (size_t)H * 4,
                                    hipMemcpyDeviceToDevice, st));
        for (anelm_hybrid_layer& L : m.layers) {
            const bool attn = L.kind == ANELM_LAYER_ATTENTION;
            const int core_dim = attn ? m.n_heads * m.head_dim : m.lin_v * m.lin_dim;
            const int first_out = attn ? m.n_heads * 2 * m.head_dim + 2 * m.n_kv_heads * m.head_dim
                                       : 2 * m.lin_k * m.lin_dim + 2 * m.lin_v * m.lin_dim + 2 * m.lin_v;
            CHECK(anelm_rmsnorm(XN, X, L.in_norm_w, H, S, H, H, m.eps, st));
            CHECK(anelm_lut6_gemm(P, L.first_w, L.first_lut, XN, S, first_out, H, 0, st));
            if (attn) {
                const float* kp = P + (size_t)m.n_heads * 2 * m.head_dim;
                CHECK(anelm_full_attn_prefill(C, P, kp, kp + (size_t)m.n_kv_heads * m.head_dim, first_out,
                                              L.k_cache, L.v_cache, L.q_norm_w, L.k_norm_w, S, m.n_heads,
                                              m.n_kv_heads, m.head_dim, m.rot_dim, L.pos, m.theta, m.eps,
                                              ANELM_ROPE_INTERLEAVED, 1, rope, m.cap, &L.cache_start, &L.cache_len,
                                              L.cache_capacity, st));
                L.pos += S;
            } else {
                CHECK(anelm_deltanet_prefill_from_proj(C, L.state, L.conv_state, &L.conv_pos, P, L.conv_w, L.dn_A,
                                                       L.dn_dt_bias, L.dn_norm_w, S, m.lin_k, m.lin_v, m.lin_dim,
                                                       m.lin_dim, m.conv_k, L.dn_flags, st));
            }
            CHECK(anelm_lut6_gemm(X, L.o_w, L.o_lut, C, S, H, core_dim, 1, st));
            CHECK(anelm_rmsnorm(XN, X, L.ffn_norm_w, H, S, H, H, m.eps, st));
            CHECK(anelm_lut6_gemm(G, L.gate_w, L.gate_lut, XN, S, I, H, 0, st));
            CHECK(anelm_lut6_gemm(U, L.up_w, L.up_lut, XN, S, I, H, 0, st));
            CHECK(anelm_swiglu(G, G, U, (int64_t)S * I, st));
            CHECK(anelm_lut6_gemm(X, L.down_w, L.down_lut, G, S, H, I, 1, st));
        }
        CHECK(anelm_rmsnorm(xf, X + (size_t)(S - 1) * H, m.final_norm, H, 1, H, H, m.eps, st));
        CHECK(anelm_lut6_gemv(logits, m.lm_w, m.lm_lut, xf, m.vocab, H, st));
    };

    if (prefill_mode == 1) {
        prefill_batch(prompt);
        // the decode step starts from the rings, positions and conv state the
        // prefill left (the step copies the descriptors)
        CHECK(anelm_hybrid_step_create(&step, &dims, m.layers.data(), m.n_layers, x, h, ANELM_STEP_EAGER, st));
    } else {
        CHECK(anelm_hybrid_step_create(&step, &dims, m.layers.data(), m.n_layers, x, h, ANELM_STEP_EAGER, st));
        for (size_t i = 0; i < prompt.size(); i++) forward(prompt[i], i + 1 == prompt.size());
    }
    std::vector<int32_t> generated;
    generated.reserve((size_t)max_tokens + 1);   // stable addresses for the async copies
    auto sample = [&]() {
        const float r = (float)rng.next();
        CHECK(anelm_sample_token(d_token, logits, m.vocab, d_recent, (int)generated.size(), temperature, rep,
                                 rep_ctx, freq, r, st));
        int32_t tok = 0;
        HIPCHECK(hipMemcpyAsync(&tok, d_token, 4, hipMemcpyDeviceToHost, st));
        HIPCHECK(hipStreamSynchronize(st));
        return (int)tok;
    };
    const auto t0 = std::chrono::steady_clock::now();
    int next = sample();
    for (int i = 0; i < max_tokens; i++) {
        generated.push_back(next);
        HIPCHECK(hipMemcpyAsync(d_recent + generated.size() - 1, &generated.back(), 4, hipMemcpyHostToDevice, st));
        printf("token %d\n", next);
        if (i + 1 == max_tokens) break;
        forward(next, true);
        next = sample();
    }
    HIPCHECK(hipStreamSynchronize(st));
    const double s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    printf("done %zu %.1f\n", generated.size(), generated.size() / (s > 0 ? s : 1e-9));
    CHECK(anelm_hybrid_step_destroy(step));
    for (void* p : g_allocs) (void)hipFree(p);
    (void)hipStreamDestroy(st);
    return 0;
}
