// Internal helpers shared by the libanelm HIP translation units: status and
// error text, the per-device workspace, and wavefront (64-lane) primitives.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>
#include <stddef.h>

#include <mutex>
#include <vector>

#include "../../include/anelm.h"

namespace anelm {

// Records a thread-local error message and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Converts a HIP status into ANELM_EHIP with the failing call named.
int hip_fail(hipError_t e, const char* what);

#define ANELM_HIP(call)                                        \
    do {                                                       \
        hipError_t e_ = (call);                                \
        if (e_ != hipSuccess) return ::anelm::hip_fail(e_, #call); \
    } while (0)

#define ANELM_REQUIRE(cond, ...)                                         \
    do {                                                                 \
        if (!(cond)) return ::anelm::set_error(ANELM_EINVAL, __VA_ARGS__); \
    } while (0)

#define ANELM_NONNULL(p)                                                      \
    do {                                                                      \
        if ((p) == nullptr) return ::anelm::set_error(ANELM_ENULL, "%s is NULL", #p); \
    } while (0)

// Launch check: reports the first launch error, if any.
#define ANELM_LAUNCHED(name)                                      \
    do {                                                          \
        hipError_t e_ = hipGetLastError();                        \
        if (e_ != hipSuccess) return ::anelm::hip_fail(e_, name); \
    } while (0)

// State of one (device, stream) pair: growable scratch buffers (contents
// undefined between calls) and a uint32 counter pool that kernels use for
// last-block-done reductions and always leave zeroed again.  Calls on
// different streams never share any of it, so they may run concurrently;
// calls on one stream are ordered by the stream.
struct StreamState {
    hipStream_t stream = nullptr;
    void* ws = nullptr;
    size_t ws_bytes = 0;
    void* ws2 = nullptr;      // second slot: split-K partials of the batched GEMM
    size_t ws2_bytes = 0;
    uint32_t* counters = nullptr;
    std::mutex mu;            // guards growth of ws / ws2
};

struct Device {
    int id = -1;
    int num_cus = 0;
    std::mutex mu;                         // guards `streams`
    std::vector<StreamState*> streams;
};

// Current device's state (lazily initialised).  nullptr on failure with the
// error recorded.
Device* device();

// State of `stream` on the current device (created on first use).
StreamState* stream_state(hipStream_t stream);
// Frees the state of `stream` on the current device (after syncing it).
int stream_release(hipStream_t stream);

// Workspace of `stream` of at least `bytes` (grows with a sync of that stream
// + free + malloc).  Returns nullptr on failure with the error recorded.
void* workspace(size_t bytes, hipStream_t stream);
// Same, from a second buffer of the stream (for callees of a workspace user).
void* workspace2(size_t bytes, hipStream_t stream);

// Workgroup barrier for LDS exchange only: this wave's LDS operations
// complete, then s_barrier.  __syncthreads() also carries a release fence that
// makes the compiler wait for every vector-memory operation of the wave
// (vmcnt(0)), which drains any global prefetch issued before the barrier.
// Use this one where the barrier only orders LDS accesses.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt unchanged
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Batched LUT6 GEMM on MFMA (lut6_mfma.hip): column split for in_dim, and the
// launch for batch <= 32 inputs.
bool lut6_gemm_geometry(int in_dim, int& np, int& waves);
int lut6_gemm_launch(float* y, const uint8_t* w, long ldw, const uint16_t* lut, const float* x, long ldx, int batch,
                     int out_dim, int in_dim, int accumulate, int nsplit, long sy, hipStream_t st);
int lut6_split_sum(float* y, const float* part, long n, int nsplit, int accumulate, hipStream_t st);
bool lut6_split_sum_norm_fits(int out_dim, int nsplit);
int lut6_split_sum_norm(float* y, const float* part, long n, int nsplit, int accumulate, int rows, int out_dim,
                        const float* norm_w, float eps, float* xn, hipStream_t st);
// Y (+)= W X over a batch (anelm_lut6_gemm), then xn = RMSNorm(Y) * norm_w per
// row: fused into the sum of the column slices where the GEMM is split.
int lut6_gemm_norm(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int batch, int out_dim,
                   int in_dim, int accumulate, const float* norm_w, float eps, float* xn, hipStream_t st);

// y (+)= W x over a LUT6 matrix, x optionally RMS-normalised first (norm_w).
int lut6_gemv_impl(float* y, const uint8_t* w, const uint16_t* lut, const float* x, const float* norm_w,
                   float eps, int out_dim, int in_dim, int residual, hipStream_t st);

// anelm_full_attn_decode with the split partials in `part` (part_cap bytes)
// instead of the library workspace when part != nullptr; and the partials
// size a call over max_len keys needs (0 for one split).
int full_attn_decode_impl(float* out, const float* q_gate, const float* k, const float* v, uint16_t* k_cache,
                          uint16_t* v_cache, const float* q_norm_w, const float* k_norm_w, int n_heads,
                          int n_kv_heads, int head_dim, int rot_dim, int pos, float theta, float eps,
                          int rope_mode, int gate, const float* cos_row, const float* sin_row, int* cache_start,
                          int* cache_len, int cache_capacity, hipStream_t stream, float* part, size_t part_cap);
size_t full_attn_part_bytes(int n_heads, int n_kv_heads, int head_dim, int max_len);
// The same over either cache element type (ANELM_F16 / ANELM_F32) and layout
// (ANELM_KV_TOKEN_MAJOR / ANELM_KV_HEAD_MAJOR).
int full_attn_decode_kv_impl(float* out, const float* q_gate, const float* k, const float* v, void* k_cache,
                             void* v_cache, int kv_dtype, int layout, const float* q_norm_w, const float* k_norm_w,
                             int n_heads, int n_kv_heads, int head_dim, int rot_dim, int pos, float theta, float eps,
                             int rope_mode, int gate, const float* cos_row, const float* sin_row, int* cache_start,
                             int* cache_len, int cache_capacity, hipStream_t stream, float* part, size_t part_cap);

// Causal prefill attention core (attn_prefill.hip): S query rows q
// [S][Hq][D] over L keys k / v [L][Hkv][D] (fp16), row r being key qoff + r
// and attending keys (qoff + r - win, qoff + r] (win 0: from key 0); out
// [S][Hq][D] fp32 or fp16; with gate, each output element is multiplied by
// sigmoid(gate[r * gtok + h * ghead + d]).  Uses the stream's workspace.
int prefill_core(void* out, bool out16, const uint16_t* q, const uint16_t* k, const uint16_t* v, int S, int L,
                 int qoff, int win, int Hq, int Hkv, int D, const float* gate, int gtok, int ghead, hipStream_t st);

// `n` counters of the pool of `stream` on the current device, in the range
// reserved for one user (ranges never overlap, so no user sees another's
// values); nullptr if n exceeds the range.  Every range starts zeroed.
enum CounterUser : int { kCtrPrefill = 0, kCtrDeltaNetConv = 1, kCtrDecode = 2, kCtrUsers = 3 };
uint32_t* counters(size_t n, CounterUser user, hipStream_t stream);

constexpr size_t kCounterPool = 1 << 16;
constexpr size_t kCounterRange = kCounterPool / 4;   // counters per user

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Host-side cos/sin for RoPE pair j at dim 2j, exactly the reference formula
// (core/cpu_ops.cpp:51-55, models/llm/qwen3_5.cpp:311-321).
void rope_row(float* cos_out, float* sin_out, int rot_dim, int pos, float theta);

constexpr int kMaxRotPairs = 128;

// Persistent decode step (step_persistent.hip): one kernel launch per step.
struct PersistentStep;
int persistent_create(PersistentStep** out, const anelm_hybrid_dims* dims,
                      const anelm_hybrid_layer* layers, int n_layers, float* x, float* h,
                      hipStream_t stream);
int persistent_run(PersistentStep* s, bool advance, bool cooperative, hipStream_t stream);
int persistent_status(PersistentStep* s, int* status);
int persistent_trace(PersistentStep* s, unsigned long long* host, size_t n_words, int* grid, int* row);
void persistent_destroy(PersistentStep* s);

// ------------------------------------------------------------- device code

__device__ __forceinline__ float h2f(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}
__device__ __forceinline__ uint16_t f2h(float f) {
    return __half_as_ushort(__float2half_rn(f));
}

// RoPE pair rotation with separately rounded products, as the reference's
// expression v0*c - v1*s evaluates without fused multiply-add
// (core/cpu_ops.cpp:57-60).
__device__ __forceinline__ void rotate_pair(float& o0, float& o1, float v0, float v1, float c,
                                            float s) {
#pragma clang fp contract(off)
    o0 = v0 * c - v1 * s;
    o1 = v0 * s + v1 * c;
}

__device__ __forceinline__ float shfl_xor(float v, int mask) {
    return __shfl_xor(v, mask, 64);
}

// Value of the stage-M exchange partner of this lane.  The partner differs
// from the lane in bit M and agrees in every bit above M:
//   M = 1, 2 : lane ^ M                     (DPP quad permute)
//   M = 4    : mirror within 8 lanes        (DPP row_half_mirror)
//   M = 8    : mirror within 16 lanes       (DPP row_mirror)
//   M = 16   : lane ^ 16 within 32 lanes    (ds_swizzle, no LDS access)
//   M = 32   : lane ^ 32                    (ds_bpermute)
// Butterfly reductions that visit M from high to low only rely on those two
// properties, so they sum exactly the same lane sets as a pure XOR butterfly.
template <int M>
__device__ __forceinline__ float partner(float v) {
    const int x = __float_as_int(v);
    int r;
    if constexpr (M == 1) r = __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, false);
    else if constexpr (M == 2) r = __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, false);
    else if constexpr (M == 4) r = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, false);
    else if constexpr (M == 8) r = __builtin_amdgcn_update_dpp(0, x, 0x140, 0xF, 0xF, false);
    else if constexpr (M == 16) r = __builtin_amdgcn_ds_swizzle(x, 0x401F);
    else r = __builtin_amdgcn_ds_bpermute((int)((__lane_id() ^ 32u) << 2), x);
    return __int_as_float(r);
}

template <int M = 32>
__device__ __forceinline__ float wave_sum_from(float v) {
    if constexpr (M >= 1) return wave_sum_from<M / 2>(v + partner<M>(v));
    return v;
}
template <int M = 32>
__device__ __forceinline__ float wave_max_from(float v) {
    if constexpr (M >= 1) return wave_max_from<M / 2>(fmaxf(v, partner<M>(v)));
    return v;
}

// Full-wave (64-lane) sum / max; every lane receives the result.
__device__ __forceinline__ float wave_sum(float v) { return wave_sum_from<32>(v); }
__device__ __forceinline__ float wave_max(float v) { return wave_max_from<32>(v); }

// Reduces R partial values held by each of L consecutive lanes (L a power of
// two <= 32, lanes aligned to L) so that lane li = lane % L ends with the
// totals of value indices (R/L)*li + j in v[j], j < R/L.  Each stage halves
// the live values: the lane keeps the half selected by its stage bit and
// adds the partner's copy of it.
template <int L, int R, int M = L / 2, int N = R>
__device__ __forceinline__ void transpose_reduce(float (&v)[R], int li) {
    static_assert(R >= L, "transpose_reduce needs R >= L");
    if constexpr (M >= 1) {
        const bool up = (li & M) != 0;
#pragma unroll
        for (int i = 0; i < N / 2; i++) {
            const float send = up ? v[i] : v[i + N / 2];
            const float keep = up ? v[i + N / 2] : v[i];
            v[i] = keep + partner<M>(send);
        }
        transpose_reduce<L, R, M / 2, N / 2>(v, li);
    }
}

// Block-wide sum for blockDim.x == NT (multiple of 64); `red` holds NT/64
// floats of shared memory.  All threads receive the total.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) t += red[i];
    return t;
}
template <int NT>
__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; i++) t = fmaxf(t, red[i]);
    return t;
}

}  // namespace anelm
