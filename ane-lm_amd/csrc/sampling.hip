// Token sampling on the device: core/sampling.cpp:11-66 (sample_token) over
// a logit vector that stays in HBM.
//
//   1. copy the logits into the adjusted buffer (the reference's memcpy, :16);
//   2. one workgroup applies the repetition / frequency penalties of the
//      distinct tokens in the last repetition_context_size entries (:18-44);
//   3. temperature <= 0: first index of the maximum (:46-53);
//      otherwise per block: scale by 1/T (:55-56) and the block maximum;
//   4. exp(x - max) and per-block sums (softmax, cpu_ops.cpp:65-75);
//   5. one workgroup: the total, the block whose running sum first reaches the
//      draw r, then the element inside it (:58-65).
// The uniform draw r is an argument (the reference calls drand48(), :57), so
// a caller owns the random stream and the result is reproducible.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

constexpr int kSNT = 256;              // threads per block
constexpr int kSPer = 8;               // elements per thread
constexpr int kSChunk = kSNT * kSPer;  // elements per block
constexpr int kSMaxWindow = 4096;      // recent tokens considered at most

__global__ __launch_bounds__(kSNT) void sample_copy_kernel(float* adj, const float* logits, int vocab) {
    const int base = blockIdx.x * kSChunk;
#pragma unroll
    for (int k = 0; k < kSPer; k++) {
        const int i = base + k * kSNT + threadIdx.x;
        if (i < vocab) adj[i] = logits[i];
    }
}

// sampling.cpp:18-44: each distinct in-range token of the window once --
// repetition penalty (divide a positive logit, multiply a non-positive one)
// if > 1, then minus frequency_penalty * count if > 0.  Thread j owns window
// entry j and acts only on the first occurrence of its token.
__global__ __launch_bounds__(kSNT) void sample_penalty_kernel(float* adj, const int32_t* recent, int start,
                                                              int n_recent, int vocab, float rep, float freq) {
    for (int j = start + threadIdx.x; j < n_recent; j += kSNT) {
        const int tok = recent[j];
        if (tok < 0 || tok >= vocab) continue;
        bool first = true;
        int count = 0;
        for (int i = start; i < n_recent; i++) {
            const int t = recent[i];
            if (t == tok) {
                if (i < j) first = false;
                count++;
            }
        }
        if (!first) continue;
        float v = adj[tok];
        if (rep > 1.0f) v = v > 0.0f ? v / rep : v * rep;
        if (freq > 0.0f) v = v - freq * (float)count;
        adj[tok] = v;
    }
}

// Block maximum with the first index attaining it (a NaN element never wins
// here: the reference's strict > never moves to one; the one exception, a NaN
// at index 0, is resolved by sample_argmax_kernel).  With scale, the values are multiplied by
// inv_t and written back first.
__global__ __launch_bounds__(kSNT) void sample_max_kernel(float* adj, float* pmax, int* pidx, int vocab,
                                                          float inv_t, int scale) {
    __shared__ float sv[kSNT / 64];
    __shared__ int si[kSNT / 64];
    const int base = blockIdx.x * kSChunk;
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int k = 0; k < kSPer; k++) {
        const int i = base + k * kSNT + threadIdx.x;
        if (i >= vocab) break;
        float v = adj[i];
        if (scale) {
            v = v * inv_t;
            adj[i] = v;
        }
        if (v > best) {
            best = v;
            bi = i;
        }
    }
    // (value desc, index asc) over the wave, then over the waves
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best, m, 64);
        const int oi = __shfl_xor(bi, m, 64);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) {
        sv[w] = best;
        si[w] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int k = 1; k < kSNT / 64; k++)
            if (sv[k] > best || (sv[k] == best && si[k] < bi)) {
                best = sv[k];
                bi = si[k];
            }
        pmax[blockIdx.x] = best;
        pidx[blockIdx.x] = bi;
    }
}

// Greedy: the first maximum over the block results (sampling.cpp:47-53).
// The reference starts from max_i = 0 and moves only on adjusted[i] >
// adjusted[max_i]: with a NaN at index 0 no comparison succeeds and it
// returns 0, whatever follows.
__global__ __launch_bounds__(64) void sample_argmax_kernel(int32_t* token, const float* adj, const float* pmax,
                                                           const int* pidx, int nb) {
    float best = -INFINITY;
    int bi = 0x7fffffff;
    for (int b = threadIdx.x; b < nb; b += 64) {
        if (pmax[b] > best || (pmax[b] == best && pidx[b] < bi)) {
            best = pmax[b];
            bi = pidx[b];
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(best, m, 64);
        const int oi = __shfl_xor(bi, m, 64);
        if (ov > best || (ov == best && oi < bi)) {
            best = ov;
            bi = oi;
        }
    }
    // every value NaN or -inf, or a NaN at index 0: the reference keeps index 0
    if (threadIdx.x == 0) *token = (bi == 0x7fffffff || __builtin_isnan(adj[0])) ? 0 : bi;
}

// Softmax numerators exp(x - max) in place and their block sums.
__global__ __launch_bounds__(kSNT) void sample_exp_kernel(float* adj, float* psum, const float* pmax, int nb,
                                                          int vocab) {
    __shared__ float red[kSNT / 64];
    float m = -INFINITY;
    for (int b = 0; b < nb; b++) m = fmaxf(m, pmax[b]);
    const int base = blockIdx.x * kSChunk;
    float s = 0.f;
    for (int k = 0; k < kSPer; k++) {
        const int i = base + k * kSNT + threadIdx.x;
        if (i >= vocab) break;
        const float e = expf(adj[i] - m);
        adj[i] = e;
        s += e;
    }
    s = block_sum<kSNT>(s, red);
    if (threadIdx.x == 0) psum[blockIdx.x] = s;
}

// One wave: the normalised running sum first reaching r (softmax multiplies by
// 1/sum, cpu_ops.cpp:72-74).  Block sums locate the block, then a wave-wide
// inclusive scan walks its elements 64 at a time; if rounding puts the
// crossing past the located block the walk continues into the next ones.
__global__ __launch_bounds__(64) void sample_draw_kernel(int32_t* token, const float* adj, const float* psum,
                                                         int nb, int vocab, float r) {
    const int lane = threadIdx.x;
    float tot = 0.f;
    for (int b = 0; b < nb; b++) tot += psum[b];   // fixed order, every lane alike
    const float inv = 1.0f / tot;
    float cum = 0.f;
    int b0 = nb - 1;
    for (int b = 0; b < nb; b++) {
        const float nxt = cum + psum[b] * inv;
        if (nxt >= r) {
            b0 = b;
            break;
        }
        cum = nxt;
    }
    int found = vocab - 1;
    for (int i0 = b0 * kSChunk; i0 < vocab; i0 += 64) {
        const int i = i0 + lane;
        float v = i < vocab ? adj[i] * inv : 0.f;
        // inclusive scan over the wave
        for (int m = 1; m < 64; m <<= 1) {
            const float o = __shfl_up(v, m, 64);
            if (lane >= m) v += o;
        }
        const float c = cum + v;
        const unsigned long long hit = __ballot(i < vocab && c >= r);
        if (hit) {
            found = i0 + __builtin_ctzll(hit);
            break;
        }
        cum += __shfl(v, 63, 64);
    }
    if (lane == 0) *token = found;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_sample_token(int32_t* token, const float* logits, int vocab, const int32_t* recent,
                                  int n_recent, float temperature, float repetition_penalty,
                                  int repetition_context_size, float frequency_penalty, float r, void* stream) {
    ANELM_NONNULL(token);
    ANELM_NONNULL(logits);
    ANELM_REQUIRE(vocab > 0, "sample_token: vocab %d", vocab);
    ANELM_REQUIRE(n_recent >= 0 && (n_recent == 0 || recent != nullptr), "sample_token: %d recent tokens",
                  n_recent);
    ANELM_REQUIRE(repetition_context_size >= 0, "sample_token: repetition context %d", repetition_context_size);
    const int start = n_recent > repetition_context_size ? n_recent - repetition_context_size : 0;
    ANELM_REQUIRE(n_recent - start <= kSMaxWindow, "sample_token: %d tokens in the penalty window (max %d)",
                  n_recent - start, kSMaxWindow);
    hipStream_t st = as_stream(stream);
    const int nb = (vocab + kSChunk - 1) / kSChunk;
    const size_t adj_n = ((size_t)vocab + 63) & ~(size_t)63;
    float* ws = static_cast<float*>(workspace((adj_n + 3 * (size_t)nb) * sizeof(float), st));
    if (!ws) return ANELM_ENOMEM;
    float* adj = ws;
    float* pmax = adj + adj_n;
    int* pidx = reinterpret_cast<int*>(pmax + nb);
    float* psum = pmax + 2 * nb;
    hipLaunchKernelGGL(sample_copy_kernel, dim3(nb), dim3(kSNT), 0, st, adj, logits, vocab);
    ANELM_LAUNCHED("sample_copy_kernel");
    if (n_recent > start) {
        hipLaunchKernelGGL(sample_penalty_kernel, dim3(1), dim3(kSNT), 0, st, adj, recent, start, n_recent, vocab,
                           repetition_penalty, frequency_penalty);
        ANELM_LAUNCHED("sample_penalty_kernel");
    }
    const bool greedy = !(temperature > 0.0f);
    hipLaunchKernelGGL(sample_max_kernel, dim3(nb), dim3(kSNT), 0, st, adj, pmax, pidx, vocab,
                       greedy ? 1.0f : 1.0f / temperature, greedy ? 0 : 1);
    ANELM_LAUNCHED("sample_max_kernel");
    if (greedy) {
        hipLaunchKernelGGL(sample_argmax_kernel, dim3(1), dim3(64), 0, st, token, adj, pmax, pidx, nb);
        ANELM_LAUNCHED("sample_argmax_kernel");
        return ANELM_OK;
    }
    hipLaunchKernelGGL(sample_exp_kernel, dim3(nb), dim3(kSNT), 0, st, adj, psum, pmax, nb, vocab);
    ANELM_LAUNCHED("sample_exp_kernel");
    hipLaunchKernelGGL(sample_draw_kernel, dim3(1), dim3(64), 0, st, token, adj, psum, nb, vocab, r);
    ANELM_LAUNCHED("sample_draw_kernel");
    return ANELM_OK;
}
