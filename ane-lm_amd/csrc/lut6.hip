// LUT6-palettised weight kernels: unpack, GEMV, fused RMSNorm + SwiGLU
// gate/up, down projection with residual, and the top-k LM head.
//
// Format: W[r][c] = lut[r/32][idx(r,c)] with a 64-entry fp16 LUT per 32-row
// group; index c of row r sits at bits [6c, 6c+6) of the row's little-endian
// byte stream (4 indices per 3 bytes, row stride in_dim*3/4 bytes).
//
// GEMV mapping: a wave owns a few rows of one 32-row group.  The row is split
// in 12-byte chunks (16 indices, dword aligned); lane l takes chunks
// l, l+64, l+128, ... so every load instruction of a wave reads 768
// contiguous bytes.  The group's 64 LUT entries live one per lane (as fp32)
// and each 6-bit index is resolved with ds_bpermute (a cross-lane read that
// needs no LDS storage and has no bank conflicts).  x is held in registers
// for the lane's chunks, so each weight costs one extract, one permute and
// one FMA.  Reference math: matvec (core/cpu_ops.cpp:77-80) on the dequantised
// weights; SwiGLU as models/llm/qwen3_5.cpp:1118-1130.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

constexpr int kNT = 256;
constexpr int kNW = kNT / 64;

__device__ __forceinline__ uint32_t idx6(const uint32_t (&w)[3], int k) {
    const int bit = 6 * k, d = bit >> 5, sh = bit & 31;
    if (sh <= 26) return (w[d] >> sh) & 63u;
    const uint64_t two = ((uint64_t)w[d + 1] << 32) | w[d];
    return (uint32_t)(two >> sh) & 63u;
}

__device__ __forceinline__ float lut_lookup(uint32_t idx, int lut_bits) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute((int)(idx << 2), lut_bits));
}

// Dot product of one 16-index chunk with 16 x values.
__device__ __forceinline__ float chunk_dot(const uint3& wv, const float* xr, int lut_bits, float acc) {
    const uint32_t w[3] = {wv.x, wv.y, wv.z};
#pragma unroll
    for (int k = 0; k < 16; k++) acc = fmaf(lut_lookup(idx6(w, k), lut_bits), xr[k], acc);
    return acc;
}

// Loads the lane's x chunks (chunks lane + 64*j) from shared memory.
template <int NJ>
__device__ __forceinline__ void load_x(float (&xr)[NJ][16], const float* xs, int nch, int lane) {
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = lane + 64 * j;
#pragma unroll
        for (int i = 0; i < 16; i++) xr[j][i] = (c < nch) ? xs[c * 16 + i] : 0.f;
    }
}

// Stages x (optionally RMS-normalised with weight nw) into shared memory.
__device__ void stage_x(float* xs, const float* x, const float* nw, float eps, int n, float* red) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kNT) {
        const float v = x[i];
        xs[i] = v;
        ss += v * v;
    }
    if (nw) {
        ss = block_sum<kNT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)n + eps);
        for (int i = threadIdx.x; i < n; i += kNT) xs[i] = (xs[i] * inv) * nw[i];
    }
    __syncthreads();
}

// Row dot products for RPW consecutive rows starting at r0 (all in one group).
template <int NJ, int RPW>
__device__ __forceinline__ void rows_dot(float (&acc)[RPW], const uint8_t* W, const uint16_t* lut,
                                         int r0, size_t row_bytes, int nch, int lane,
                                         const float (&xr)[NJ][16]) {
    const int lut_bits = __float_as_int(h2f(lut[(size_t)(r0 >> 5) * 64 + lane]));
    uint3 wv[RPW][NJ];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int c = lane + 64 * j;
            wv[r][j] = (c < nch) ? *reinterpret_cast<const uint3*>(W + (size_t)(r0 + r) * row_bytes + (size_t)c * 12)
                                 : make_uint3(0u, 0u, 0u);
        }
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++) a = chunk_dot(wv[r][j], xr[j], lut_bits, a);
        acc[r] = wave_sum(a);
    }
}

// y[r] = (residual ? y[r] : 0) + W x.  Rows per workgroup = 4 * RPW.
template <int NJ, int RPW>
__global__ __launch_bounds__(kNT) void lut6_gemv_kernel(float* y, const uint8_t* W, const uint16_t* lut,
                                                        const float* x, int out_dim, int in_dim,
                                                        int residual) {
    extern __shared__ float xs[];
    __shared__ float red[kNW];
    stage_x(xs, x, nullptr, 0.f, in_dim, red);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * kNW + w) * RPW;
    if (r0 >= out_dim) return;
    const int nch = in_dim / 16;
    float xr[NJ][16];
    load_x<NJ>(xr, xs, nch, lane);
    float acc[RPW];
    rows_dot<NJ, RPW>(acc, W, lut, r0, (size_t)in_dim * 3 / 4, nch, lane, xr);
    if (lane < RPW) {
        float v = acc[0];
#pragma unroll
        for (int r = 1; r < RPW; r++) if (lane == r) v = acc[r];
        y[r0 + lane] = residual ? y[r0 + lane] + v : v;
    }
}

// h[r] = silu(gate_r . n) * (up_r . n), n = rmsnorm(x, nw) (or x when nw is NULL).
template <int NJ, int RPW>
__global__ __launch_bounds__(kNT) void lut6_gateup_kernel(float* h, const uint8_t* Wg, const uint16_t* lg,
                                                          const uint8_t* Wu, const uint16_t* lu,
                                                          const float* x, const float* nw, float eps,
                                                          int inter, int hidden) {
    extern __shared__ float xs[];
    __shared__ float red[kNW];
    stage_x(xs, x, nw, eps, hidden, red);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r0 = (blockIdx.x * kNW + w) * RPW;
    if (r0 >= inter) return;
    const int nch = hidden / 16;
    const size_t rb = (size_t)hidden * 3 / 4;
    float xr[NJ][16];
    load_x<NJ>(xr, xs, nch, lane);
    float ag[RPW], au[RPW];
    rows_dot<NJ, RPW>(ag, Wg, lg, r0, rb, nch, lane, xr);
    rows_dot<NJ, RPW>(au, Wu, lu, r0, rb, nch, lane, xr);
    if (lane < RPW) {
        float g = ag[0], u = au[0];
#pragma unroll
        for (int r = 1; r < RPW; r++) if (lane == r) { g = ag[r]; u = au[r]; }
        h[r0 + lane] = (g / (1.0f + expf(-g))) * u;
    }
}

__global__ void lut6_unpack_kernel(uint8_t* idx, const uint8_t* packed, int64_t groups) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= groups) return;
    const uint32_t b0 = packed[3 * g], b1 = packed[3 * g + 1], b2 = packed[3 * g + 2];
    const uint32_t w = b0 | (b1 << 8) | (b2 << 16);
    uchar4 o;
    o.x = (uint8_t)(w & 63u);
    o.y = (uint8_t)((w >> 6) & 63u);
    o.z = (uint8_t)((w >> 12) & 63u);
    o.w = (uint8_t)((w >> 18) & 63u);
    *reinterpret_cast<uchar4*>(idx + 4 * g) = o;
}

// ---------------------------------------------------------------- top-k
// Ordering (value desc, index asc): a precedes b.
__device__ __forceinline__ bool before(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

constexpr int kTopkChunk = 2048;   // logits per selection workgroup

// Bitonic sort of n (power of two) (value, index) pairs in shared memory,
// best first.
__device__ void bitonic_sort(float* v, int* id, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            __syncthreads();
            for (int t = threadIdx.x; t < n / 2; t += kNT) {
                const int lo = 2 * t - (t & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const bool swap = desc ? before(v[hi], id[hi], v[lo], id[lo])
                                       : before(v[lo], id[lo], v[hi], id[hi]);
                if (swap) {
                    const float tv = v[lo]; v[lo] = v[hi]; v[hi] = tv;
                    const int ti = id[lo]; id[lo] = id[hi]; id[hi] = ti;
                }
            }
        }
    }
    __syncthreads();
}

// Stage 1: each workgroup sorts one chunk of one batch row's logits and keeps
// the best k as candidates [batch][n_chunks][k].
__global__ __launch_bounds__(kNT) void topk_stage1(const float* logits, int n, int k, int n_chunks,
                                                   float* cv, int* ci) {
    __shared__ float v[kTopkChunk];
    __shared__ int id[kTopkChunk];
    const int chunk = blockIdx.x, b = blockIdx.y;
    const int base = chunk * kTopkChunk;
    for (int t = threadIdx.x; t < kTopkChunk; t += kNT) {
        const int r = base + t;
        v[t] = (r < n) ? logits[(size_t)b * n + r] : -INFINITY;
        id[t] = (r < n) ? r : 0x7fffffff;
    }
    bitonic_sort(v, id, kTopkChunk);
    for (int t = threadIdx.x; t < k; t += kNT) {
        cv[((size_t)b * n_chunks + chunk) * k + t] = v[t];
        ci[((size_t)b * n_chunks + chunk) * k + t] = id[t];
    }
}

// Stage 2: one workgroup per batch row sorts all candidates (padded to a
// power of two) and writes the best k.
__global__ __launch_bounds__(kNT) void topk_stage2(const float* cv, const int* ci, int n_cand, int np2,
                                                   int k, int32_t* out_idx, float* out_val) {
    extern __shared__ float sm[];
    float* v = sm;
    int* id = reinterpret_cast<int*>(sm + np2);
    const int b = blockIdx.x;
    for (int t = threadIdx.x; t < np2; t += kNT) {
        v[t] = (t < n_cand) ? cv[(size_t)b * n_cand + t] : -INFINITY;
        id[t] = (t < n_cand) ? ci[(size_t)b * n_cand + t] : 0x7fffffff;
    }
    bitonic_sort(v, id, np2);
    for (int t = threadIdx.x; t < k; t += kNT) {
        out_idx[(size_t)b * k + t] = id[t];
        out_val[(size_t)b * k + t] = v[t];
    }
}

constexpr int kMaxNJ = 16;   // in_dim up to 16384

template <int NJ>
int gemv_nj(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int out_dim,
            int in_dim, int residual, hipStream_t st) {
    constexpr int RPW = (NJ <= 4) ? 4 : 2;
    const int rows_per_block = kNW * RPW;
    const int blocks = (out_dim + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((lut6_gemv_kernel<NJ, RPW>), dim3(blocks), dim3(kNT),
                       (size_t)in_dim * sizeof(float), st, y, w, lut, x, out_dim, in_dim, residual);
    ANELM_LAUNCHED("lut6_gemv_kernel");
    return ANELM_OK;
}

template <int NJ>
int gateup_nj(float* h, const uint8_t* wg, const uint16_t* lg, const uint8_t* wu,
              const uint16_t* lu, const float* x, const float* nw, float eps, int inter,
              int hidden, hipStream_t st) {
    constexpr int RPW = (NJ <= 4) ? 4 : 2;
    const int rows_per_block = kNW * RPW;
    const int blocks = (inter + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((lut6_gateup_kernel<NJ, RPW>), dim3(blocks), dim3(kNT),
                       (size_t)hidden * sizeof(float), st, h, wg, lg, wu, lu, x, nw, eps, inter,
                       hidden);
    ANELM_LAUNCHED("lut6_gateup_kernel");
    return ANELM_OK;
}

int gemv_dispatch(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int out_dim,
                  int in_dim, int residual, hipStream_t st) {
    const int nj = (in_dim / 16 + 63) / 64;
    switch (nj) {
#define CASE(N) case N: return gemv_nj<N>(y, w, lut, x, out_dim, in_dim, residual, st);
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
        CASE(9) CASE(10) CASE(11) CASE(12) CASE(13) CASE(14) CASE(15) CASE(16)
#undef CASE
        default: return set_error(ANELM_ERANGE, "lut6: in_dim %d beyond %d", in_dim, kMaxNJ * 1024);
    }
}

int gateup_dispatch(float* h, const uint8_t* wg, const uint16_t* lg, const uint8_t* wu,
                    const uint16_t* lu, const float* x, const float* nw, float eps, int inter,
                    int hidden, hipStream_t st) {
    const int nj = (hidden / 16 + 63) / 64;
    switch (nj) {
#define CASE(N) case N: return gateup_nj<N>(h, wg, lg, wu, lu, x, nw, eps, inter, hidden, st);
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8)
        CASE(9) CASE(10) CASE(11) CASE(12) CASE(13) CASE(14) CASE(15) CASE(16)
#undef CASE
        default: return set_error(ANELM_ERANGE, "lut6: hidden %d beyond %d", hidden, kMaxNJ * 1024);
    }
}

int check_shape(int out_dim, int in_dim) {
    ANELM_REQUIRE(out_dim > 0 && out_dim % 32 == 0, "lut6: out_dim %d must be a positive multiple of 32", out_dim);
    ANELM_REQUIRE(in_dim > 0 && in_dim % 16 == 0, "lut6: in_dim %d must be a positive multiple of 16", in_dim);
    ANELM_REQUIRE(in_dim <= kMaxNJ * 1024, "lut6: in_dim %d beyond %d", in_dim, kMaxNJ * 1024);
    return ANELM_OK;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" {

int anelm_lut6_unpack(uint8_t* idx, const uint8_t* packed, int64_t n, void* stream) {
    ANELM_NONNULL(idx);
    ANELM_NONNULL(packed);
    ANELM_REQUIRE(n >= 0 && n % 4 == 0, "lut6_unpack: n %lld must be a multiple of 4", (long long)n);
    const int64_t groups = n / 4;
    if (groups == 0) return ANELM_OK;
    hipLaunchKernelGGL(lut6_unpack_kernel, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0,
                       as_stream(stream), idx, packed, groups);
    ANELM_LAUNCHED("lut6_unpack_kernel");
    return ANELM_OK;
}

int anelm_lut6_gemv(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int out_dim,
                    int in_dim, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(w);
    ANELM_NONNULL(lut);
    ANELM_NONNULL(x);
    int rc = check_shape(out_dim, in_dim);
    if (rc) return rc;
    return gemv_dispatch(y, w, lut, x, out_dim, in_dim, 0, as_stream(stream));
}

int anelm_lut6_ffn(float* x, float* h_scratch, const float* norm_w, float eps,
                   const uint8_t* gate_w, const uint16_t* gate_lut, const uint8_t* up_w,
                   const uint16_t* up_lut, const uint8_t* down_w, const uint16_t* down_lut,
                   int hidden, int inter, void* stream) {
    ANELM_NONNULL(x);
    ANELM_NONNULL(h_scratch);
    ANELM_NONNULL(gate_w);
    ANELM_NONNULL(gate_lut);
    ANELM_NONNULL(up_w);
    ANELM_NONNULL(up_lut);
    ANELM_NONNULL(down_w);
    ANELM_NONNULL(down_lut);
    int rc = check_shape(inter, hidden);
    if (rc) return rc;
    rc = check_shape(hidden, inter);
    if (rc) return rc;
    hipStream_t st = as_stream(stream);
    rc = gateup_dispatch(h_scratch, gate_w, gate_lut, up_w, up_lut, x, norm_w, eps, inter, hidden, st);
    if (rc) return rc;
    return gemv_dispatch(x, down_w, down_lut, h_scratch, hidden, inter, 1, st);
}

int anelm_lut6_swiglu(float* h, const float* x, const float* norm_w, float eps,
                      const uint8_t* gate_w, const uint16_t* gate_lut, const uint8_t* up_w,
                      const uint16_t* up_lut, int hidden, int inter, void* stream) {
    ANELM_NONNULL(h);
    ANELM_NONNULL(x);
    ANELM_NONNULL(gate_w);
    ANELM_NONNULL(gate_lut);
    ANELM_NONNULL(up_w);
    ANELM_NONNULL(up_lut);
    int rc = check_shape(inter, hidden);
    if (rc) return rc;
    return gateup_dispatch(h, gate_w, gate_lut, up_w, up_lut, x, norm_w, eps, inter, hidden,
                           as_stream(stream));
}

int anelm_lut6_topk(int32_t* out_idx, float* out_val, const uint8_t* w, const uint16_t* lut,
                    const float* x, int batch, int out_dim, int in_dim, int k, void* stream) {
    ANELM_NONNULL(out_idx);
    ANELM_NONNULL(out_val);
    ANELM_NONNULL(w);
    ANELM_NONNULL(lut);
    ANELM_NONNULL(x);
    int rc = check_shape(out_dim, in_dim);
    if (rc) return rc;
    ANELM_REQUIRE(batch > 0, "lut6_topk: batch %d", batch);
    ANELM_REQUIRE(k > 0 && k <= 64 && k <= out_dim, "lut6_topk: k %d must be in [1, min(64, out_dim)]", k);
    hipStream_t st = as_stream(stream);
    const int n_chunks = (out_dim + kTopkChunk - 1) / kTopkChunk;
    const int n_cand = n_chunks * k;
    int np2 = 1;
    while (np2 < n_cand) np2 <<= 1;
    ANELM_REQUIRE(np2 <= 8192, "lut6_topk: %d candidates exceed the merge limit", n_cand);
    const size_t logits_bytes = (size_t)batch * out_dim * sizeof(float);
    const size_t cand_bytes = (size_t)batch * n_cand * (sizeof(float) + sizeof(int));
    char* ws = static_cast<char*>(workspace(logits_bytes + cand_bytes, st));
    if (!ws) return ANELM_ENOMEM;
    float* logits = reinterpret_cast<float*>(ws);
    float* cv = reinterpret_cast<float*>(ws + logits_bytes);
    int* ci = reinterpret_cast<int*>(ws + logits_bytes + (size_t)batch * n_cand * sizeof(float));
    for (int b = 0; b < batch; b++) {
        rc = gemv_dispatch(logits + (size_t)b * out_dim, w, lut, x + (size_t)b * in_dim, out_dim,
                           in_dim, 0, st);
        if (rc) return rc;
    }
    hipLaunchKernelGGL(topk_stage1, dim3(n_chunks, batch), dim3(kNT), 0, st, logits, out_dim, k,
                       n_chunks, cv, ci);
    ANELM_LAUNCHED("topk_stage1");
    hipLaunchKernelGGL(topk_stage2, dim3(batch), dim3(kNT), (size_t)np2 * 8, st, cv, ci, n_cand,
                       np2, k, out_idx, out_val);
    ANELM_LAUNCHED("topk_stage2");
    return ANELM_OK;
}

}  // extern "C"
