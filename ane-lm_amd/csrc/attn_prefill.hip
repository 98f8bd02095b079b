// Causal GQA prefill attention on fp16 MFMA (v_mfma_f32_32x32x16_f16) with
// fp32 accumulation and an online softmax.
//
// Reference semantics: the reference has no batched prefill; generate.cpp:76-84
// runs the decode core once per prompt token, so output row t is
// gqa_attention (core/cpu_ops.cpp:148-204) over keys 0..t.
//
// Formulation: each wave owns 32 query rows of one head and computes the
// transposed score tile S^T = K Q^T (32 keys x 32 rows), so that in the MFMA
// accumulator layout every lane holds 16 scores of ONE query row.  The row's
// softmax statistics therefore need one cross-half exchange only, the output
// rescale is a per-lane scalar, and P^T is already in the B-operand layout of
// the second product O^T += V^T P^T (the contraction order over keys is
// permuted identically in both operands).  K and V^T tiles of 32 keys are
// staged in LDS once per workgroup and shared by all waves (the query heads of
// one KV head and several row blocks).
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float float16_t __attribute__((ext_vector_type(16)));

constexpr int kBN = 32;  // keys per tile

template <int D, int HB, int RB, bool OUT16>
__global__ __launch_bounds__(HB * RB * 64) void prefill_kernel(void* out, const _Float16* q,
                                                               const _Float16* k, const _Float16* v,
                                                               int S, int Hq, int Hkv) {
    constexpr int NW = HB * RB;
    constexpr int NT = NW * 64;
    constexpr int KS = D / 16;   // QK k-steps
    constexpr int DB = D / 32;   // PV dim blocks
    constexpr int KP = D + 8;    // K tile row pitch (halfs): 16-byte aligned rows, conflict-free reads
    constexpr int VP = kBN + 4;  // V^T row pitch (halfs)
    __shared__ __attribute__((aligned(16))) _Float16 Ks[kBN][KP];
    __shared__ __attribute__((aligned(16))) _Float16 Vt[D][VP];

    const int G = Hq / Hkv;
    const int qt = gridDim.x - 1 - blockIdx.x;  // longest causal ranges first
    const int h0 = blockIdx.y * HB;
    const int kvh = h0 / G;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int h = h0 + (w % HB);
    const int q0 = (qt * RB + w / HB) * 32;
    const int row_end = min(S, (qt + 1) * RB * 32);
    const int r = lane & 31, hh = lane >> 5;
    const int qrow = q0 + r;

    half8 qf[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ks++) {
        if (qrow < S) qf[ks] = *reinterpret_cast<const half8*>(q + ((size_t)qrow * Hq + h) * D + 16 * ks + 8 * hh);
        else qf[ks] = half8{};
    }

    float16_t o[DB];
#pragma unroll
    for (int db = 0; db < DB; db++) o[db] = float16_t{};
    float m = -INFINITY, l = 0.f;
    const float sl2 = (1.0f / sqrtf((float)D)) * 1.4426950408889634f;

    const int nkt = (row_end + kBN - 1) / kBN;
    for (int kt = 0; kt < nkt; kt++) {
        const int j0 = kt * kBN;
        __syncthreads();
        for (int c = tid; c < kBN * D / 8; c += NT) {
            const int kr = c / (D / 8), kc = (c % (D / 8)) * 8;
            const int key = j0 + kr;
            uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
            if (key < S) {
                kv4 = *reinterpret_cast<const uint4*>(k + ((size_t)key * Hkv + kvh) * D + kc);
                vv4 = *reinterpret_cast<const uint4*>(v + ((size_t)key * Hkv + kvh) * D + kc);
            }
            *reinterpret_cast<uint4*>(&Ks[kr][kc]) = kv4;
            const _Float16* vh = reinterpret_cast<const _Float16*>(&vv4);
#pragma unroll
            for (int i = 0; i < 8; i++) Vt[kc + i][kr] = vh[i];
        }
        __syncthreads();
        if (q0 >= S || j0 > q0 + 31) continue;  // wave-uniform: tile fully masked

        float16_t s = float16_t{};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const half8 a = *reinterpret_cast<const half8*>(&Ks[r][16 * ks + 8 * hh]);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], s, 0, 0, 0);
        }
        // s[e] = score of key j0 + 8*(e/4) + 4*hh + e%4 for query row qrow
        float mx = -INFINITY;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int key = j0 + 8 * (e / 4) + 4 * hh + (e % 4);
            const float val = (key <= qrow) ? s[e] * sl2 : -INFINITY;
            s[e] = val;
            mx = fmaxf(mx, val);
        }
        mx = fmaxf(mx, shfl_xor(mx, 32));
        const float m_new = fmaxf(m, mx);
        const float alpha = exp2f(m - m_new);
        float ps = 0.f;
        half8 pf[2];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const float pe = exp2f(s[e] - m_new);
            ps += pe;
            pf[e / 8][e % 8] = (_Float16)pe;
        }
        l = l * alpha + ps;
        m = m_new;
#pragma unroll
        for (int db = 0; db < DB; db++) {
#pragma unroll
            for (int e = 0; e < 16; e++) o[db][e] *= alpha;
#pragma unroll
            for (int kk = 0; kk < 2; kk++) {
                const half4 lo = *reinterpret_cast<const half4*>(&Vt[32 * db + r][16 * kk + 4 * hh]);
                const half4 hi = *reinterpret_cast<const half4*>(&Vt[32 * db + r][16 * kk + 8 + 4 * hh]);
                const half8 a = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pf[kk], o[db], 0, 0, 0);
            }
        }
    }
    if (q0 >= S) return;
    l += shfl_xor(l, 32);
    if (qrow >= S) return;
    const float inv = 1.0f / l;
    // o[db][e] = output dim 32*db + 8*(e/4) + 4*hh + e%4 of row qrow
#pragma unroll
    for (int db = 0; db < DB; db++) {
#pragma unroll
        for (int g4 = 0; g4 < 4; g4++) {
            const int d = 32 * db + 8 * g4 + 4 * hh;
            const size_t off = ((size_t)qrow * Hq + h) * D + d;
            const float a0 = o[db][4 * g4] * inv, a1 = o[db][4 * g4 + 1] * inv;
            const float a2 = o[db][4 * g4 + 2] * inv, a3 = o[db][4 * g4 + 3] * inv;
            if (OUT16) {
                half4 hv = {(_Float16)a0, (_Float16)a1, (_Float16)a2, (_Float16)a3};
                *reinterpret_cast<half4*>(static_cast<_Float16*>(out) + off) = hv;
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(out) + off) = make_float4(a0, a1, a2, a3);
            }
        }
    }
}

template <int D, int HB, int RB>
int launch_prefill(void* out, bool out16, const void* q, const void* k, const void* v, int S, int Hq,
                   int Hkv, hipStream_t st) {
    const int rows = 32 * RB;
    dim3 grid((S + rows - 1) / rows, Hq / HB), block(HB * RB * 64);
    const _Float16* qh = static_cast<const _Float16*>(q);
    const _Float16* kh = static_cast<const _Float16*>(k);
    const _Float16* vh = static_cast<const _Float16*>(v);
    if (out16) hipLaunchKernelGGL((prefill_kernel<D, HB, RB, true>), grid, block, 0, st, out, qh, kh, vh, S, Hq, Hkv);
    else hipLaunchKernelGGL((prefill_kernel<D, HB, RB, false>), grid, block, 0, st, out, qh, kh, vh, S, Hq, Hkv);
    ANELM_LAUNCHED("prefill_kernel");
    return ANELM_OK;
}

template <int D>
int dispatch_g(void* out, bool out16, const void* q, const void* k, const void* v, int S, int Hq,
               int Hkv, hipStream_t st) {
    switch (Hq / Hkv) {
        case 1: return launch_prefill<D, 1, 8>(out, out16, q, k, v, S, Hq, Hkv, st);
        case 2: return launch_prefill<D, 2, 4>(out, out16, q, k, v, S, Hq, Hkv, st);
        case 4: return launch_prefill<D, 4, 2>(out, out16, q, k, v, S, Hq, Hkv, st);
        case 8: return launch_prefill<D, 4, 2>(out, out16, q, k, v, S, Hq, Hkv, st);
        default: return set_error(ANELM_EINVAL, "prefill: n_heads/n_kv_heads = %d unsupported", Hq / Hkv);
    }
}

}  // namespace
}  // namespace anelm

using namespace anelm;

extern "C" int anelm_attn_prefill(void* out, int out_dtype, const uint16_t* q, const uint16_t* k,
                                  const uint16_t* v, int S, int n_heads, int n_kv_heads,
                                  int head_dim, void* stream) {
    ANELM_NONNULL(out);
    ANELM_NONNULL(q);
    ANELM_NONNULL(k);
    ANELM_NONNULL(v);
    ANELM_REQUIRE(S > 0, "prefill: S %d", S);
    ANELM_REQUIRE(n_kv_heads > 0 && n_heads % n_kv_heads == 0, "prefill: heads %d/%d", n_heads,
                  n_kv_heads);
    ANELM_REQUIRE(out_dtype == ANELM_F32 || out_dtype == ANELM_F16, "prefill: out_dtype %d", out_dtype);
    const bool out16 = out_dtype == ANELM_F16;
    hipStream_t st = as_stream(stream);
    switch (head_dim) {
        case 128: return dispatch_g<128>(out, out16, q, k, v, S, n_heads, n_kv_heads, st);
        case 256: return dispatch_g<256>(out, out16, q, k, v, S, n_heads, n_kv_heads, st);
        default: return set_error(ANELM_EINVAL, "prefill: head_dim %d unsupported (128, 256)", head_dim);
    }
}
