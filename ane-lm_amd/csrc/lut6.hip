// LUT6-palettised weight kernels: unpack, GEMV, the FFN block (RMSNorm +
// gate/up + SwiGLU + down + residual), and the top-k LM head.
//
// Format: W[r][c] = lut[r/32][idx(r,c)] with a 64-entry fp16 LUT per 32-row
// group; index c of row r sits at bits [6c, 6c+6) of the row's little-endian
// byte stream (4 indices per 3 bytes, row stride in_dim*3/4 bytes).
//
// GEMV mapping.  A workgroup (4 waves) owns 4*RPW rows of ONE 32-row group.
// A row is split into 12-byte chunks (16 indices, dword aligned); lane l takes
// chunks l, l+64, l+128, ... so every load instruction of a wave reads 768
// contiguous bytes.  The weight loads are issued first, so their latency is
// covered by the rest of the prologue: staging x into LDS (with the fused
// RMSNorm or SwiGLU) and building the group's pair table -- 4096 float2
// entries T[(i1 << 6) | i0] = (lut[i0], lut[i1]).  Two adjacent 6-bit indices
// are one contiguous 12-bit field of the row stream, so one extract and one
// 8-byte LDS read dequantise two weights.  Reference math: matvec
// (core/cpu_ops.cpp:77-80) on the dequantised weights; SwiGLU as
// models/llm/qwen3_5.cpp:1118-1130.
#include "anelm_internal.hpp"

#include <math.h>

namespace anelm {
namespace {

constexpr int kNT = 256;
constexpr int kNW = kNT / 64;
constexpr int kPairs = 4096;

// Bit-field [bit, bit+n) of the 96-bit chunk (w0 | w1<<32 | w2<<64).
template <int BIT, int N>
__device__ __forceinline__ uint32_t field(uint32_t w0, uint32_t w1, uint32_t w2) {
    constexpr int d = BIT >> 5, sh = BIT & 31;
    const uint32_t lo = d == 0 ? w0 : (d == 1 ? w1 : w2);
    if constexpr (sh + N <= 32) {
        return (lo >> sh) & ((1u << N) - 1u);
    } else {
        const uint32_t hi = d == 0 ? w1 : w2;
        return __builtin_amdgcn_alignbit(hi, lo, sh) & ((1u << N) - 1u);
    }
}

// Builds the pair table of LUT group `lut64` in shared memory: entry
// (i1 << 6) | i0 holds lut[i0] in its low half and lut[i1] in its high half.
__device__ __forceinline__ void build_pairs(uint32_t* tab, const uint16_t* lut64) {
    for (int e = threadIdx.x; e < kPairs; e += kNT)
        tab[e] = (uint32_t)lut64[e & 63] | ((uint32_t)lut64[e >> 6] << 16);
}

__device__ __forceinline__ float lo_half(uint32_t p) {
    return __half2float(__ushort_as_half((unsigned short)(p & 0xffffu)));
}
__device__ __forceinline__ float hi_half(uint32_t p) {
    return __half2float(__ushort_as_half((unsigned short)(p >> 16)));
}

// Dot product of one 16-index chunk with its 16 x values (fp16 weights
// widened exactly; fp32 products and sums).
__device__ __forceinline__ void chunk_dot(const uint32_t* tab, uint32_t w0, uint32_t w1, uint32_t w2,
                                          const float (&xr)[16], float& a0, float& a1) {
    uint32_t p[8];
    p[0] = tab[field<0, 12>(w0, w1, w2)];
    p[1] = tab[field<12, 12>(w0, w1, w2)];
    p[2] = tab[field<24, 12>(w0, w1, w2)];
    p[3] = tab[field<36, 12>(w0, w1, w2)];
    p[4] = tab[field<48, 12>(w0, w1, w2)];
    p[5] = tab[field<60, 12>(w0, w1, w2)];
    p[6] = tab[field<72, 12>(w0, w1, w2)];
    p[7] = tab[field<84, 12>(w0, w1, w2)];
#pragma unroll
    for (int k = 0; k < 8; k++) {
        a0 = fmaf(lo_half(p[k]), xr[2 * k], a0);
        a1 = fmaf(hi_half(p[k]), xr[2 * k + 1], a1);
    }
}

// x staging modes
enum : int { kStageCopy = 0, kStageNorm = 1, kStageSwiglu = 2 };

// Stages the GEMV input vector into shared memory:
//   copy:   xs = x
//   norm:   xs = rmsnorm(x, nw, eps)           (cpu_ops.cpp:24-30)
//   swiglu: xs = silu(x) * x2                  (qwen3_5.cpp:1123-1126)
// then rounded to fp16 (the LUT6 matrices take fp16 activations).
template <int MODE>
__device__ void stage_x(float* xs, const float* x, const float* x2, const float* nw, float eps, int n,
                        float* red) {
    if (MODE == kStageSwiglu) {
        for (int i = threadIdx.x; i < n; i += kNT) {
            const float g = x[i];
            xs[i] = (float)(_Float16)((g / (1.0f + expf(-g))) * x2[i]);
        }
        return;
    }
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += kNT) {
        const float v = x[i];
        xs[i] = v;
        ss += v * v;
    }
    if (MODE == kStageNorm && nw != nullptr) {
        ss = block_sum<kNT>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)n + eps);
        for (int i = threadIdx.x; i < n; i += kNT) xs[i] = (float)(_Float16)((xs[i] * inv) * nw[i]);
    } else {
        for (int i = threadIdx.x; i < n; i += kNT) xs[i] = (float)(_Float16)xs[i];
    }
}

struct GemvArgs {
    // up to two matrices sharing the input: blocks [0, blocks0) use matrix 0
    const uint8_t* w[2];
    const uint16_t* lut[2];
    float* y[2];
    int blocks0;
    int out_dim, in_dim;
    const float* x;
    const float* x2;       // swiglu second operand
    const float* nw;       // rmsnorm weight
    float eps;
    int residual;          // y[r] += result instead of y[r] = result
};

// Rows [r0, r0 + 4*RPW) of one matrix; one 32-row LUT group per workgroup.
template <int NJ, int RPW, int STAGE>
__global__ __launch_bounds__(kNT) void lut6_gemv_kernel(const GemvArgs a) {
    static_assert(kNW * RPW <= 32, "a workgroup must stay inside one LUT group");
    extern __shared__ float smem[];
    uint32_t* tab = reinterpret_cast<uint32_t*>(smem);
    float* xs = smem + kPairs;
    __shared__ float red[kNW];

    const int m = blockIdx.x < a.blocks0 ? 0 : 1;
    const int blk = m == 0 ? blockIdx.x : blockIdx.x - a.blocks0;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int rb0 = blk * kNW * RPW;             // first row of the workgroup
    const int r0 = rb0 + w * RPW;                // first row of this wave
    const int nch = a.in_dim / 16;
    const size_t row_bytes = (size_t)a.in_dim * 3 / 4;
    const uint8_t* W = a.w[m];

    // 1. weight loads first
    uint32_t wv[RPW][NJ][3];
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int j = 0; j < NJ; j++) {
            const int c = lane + 64 * j;
            uint3 t = make_uint3(0u, 0u, 0u);
            if (c < nch) t = *reinterpret_cast<const uint3*>(W + (size_t)(r0 + r) * row_bytes + (size_t)c * 12);
            wv[r][j][0] = t.x;
            wv[r][j][1] = t.y;
            wv[r][j][2] = t.z;
        }
    // 2. pair table and staged x while the weights are in flight
    build_pairs(tab, a.lut[m] + (size_t)(rb0 >> 5) * 64);
    stage_x<STAGE>(xs, a.x, a.x2, a.nw, a.eps, a.in_dim, red);
    __syncthreads();
    float xr[NJ][16];
#pragma unroll
    for (int j = 0; j < NJ; j++) {
        const int c = lane + 64 * j;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
            if (c < nch) v = reinterpret_cast<const float4*>(xs + c * 16)[q];
            xr[j][4 * q] = v.x;
            xr[j][4 * q + 1] = v.y;
            xr[j][4 * q + 2] = v.z;
            xr[j][4 * q + 3] = v.w;
        }
    }
    // 3. dot products
    float res = 0.f;
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float a0 = 0.f, a1 = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; j++) chunk_dot(tab, wv[r][j][0], wv[r][j][1], wv[r][j][2], xr[j], a0, a1);
        const float s = wave_sum(a0 + a1);
        if (lane == r) res = s;
    }
    if (lane < RPW) {
        float* y = a.y[m] + r0 + lane;
        *y = a.residual ? *y + res : res;
    }
}

// ------------------------------------------------------- tile GEMV (fast path)
//
// Geometry.  A row holds C = in_dim/16 chunks of 12 bytes; a tile of T rows
// is T*C contiguous chunks.  One wave instruction reads 64 consecutive
// chunks (768 bytes).  With P = C / gcd(C, 64) waves per matrix, wave w of a
// matrix issues instructions w, w+P, w+2P, ... of the tile, so lane l always
// sees the same chunk position pos = (64w + l) % C, on row RP*m + d of
// instruction m, where RP = 64P/C and d = (64w + l) / C.  Every lane
// therefore needs the 16 x values of ONE chunk for the whole tile: they sit
// in registers as fp16 pairs -- the LUT6 matrices take fp16 activations, as
// the reference's CoreML models do (core/coreml_runtime.cpp:331-336) -- and
// v_dot2_f32_f16 dots two weights with two x values, accumulating in fp32
// (fp16 products are exact in fp32).  A 12-bit index pair selects one dword of the LDS pair
// table T[(i1 << 6) | i0] = lut[i0] | lut[i1] << 16, built from the group's
// LUT held one entry per lane.  Partial sums are reduced through LDS in a
// fixed order, so results are deterministic.
//
// A workgroup has NMAT * P waves: NMAT = 2 runs gate and up over the same
// rows (same geometry, one pair table each) so the SwiGLU product
// (qwen3_5.cpp:1123-1126) is formed in the epilogue.  The small loads (LUT,
// x, norm weight) are issued before the weight stream, because vector memory
// waits complete in order.

// Output modes of the tile kernel.
enum : int { kOutY = 0, kOutGU = 1, kOutH = 2 };

struct TileArgs {
    const uint8_t* w[2];
    const uint16_t* lut[2];
    float* y[2];          // kOutY: y[0]; kOutGU: g = y[0], u = y[1]; kOutH: h = y[0]
    const float* x;
    const float* nw;      // RMSNorm weight (NULL: no norm)
    float eps;
    int n_mat;            // 1 or 2
    int mode;             // kOut*
    int residual;         // kOutY: y += W x
    int in_dim, C, P, RP, T;
    int tpr;              // reduction threads per row (power of two <= 64)
};

// LDS byte offset of the pair-table entry addressed by the 12-bit field at
// bit B of the 96-bit chunk, OR-ed with the table base `tb` (bit 14).
template <int B>
__device__ __forceinline__ uint32_t pair_addr(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t tb) {
    uint32_t v;
    if constexpr (B == 0) {
        v = w0 << 2;
    } else {
        constexpr int s = B - 2, d = s >> 5, sh = s & 31;
        const uint32_t lo = d == 0 ? w0 : (d == 1 ? w1 : w2);
        const uint32_t hi = d == 0 ? w1 : w2;
        v = (sh + 14 <= 32) ? (lo >> sh) : __builtin_amdgcn_alignbit(hi, lo, sh);
    }
    return (v & 0x3FFCu) | tb;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// Word 3 of a raw (unformatted, stride 0) buffer descriptor on gfx9-class GPUs.
constexpr int kBufferRsrcWord3 = 0x00020000;

__device__ __forceinline__ float dot2(uint32_t p, uint32_t x, float acc) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(half2_t, p), __builtin_bit_cast(half2_t, x), acc,
                                  false);
}

__device__ __forceinline__ uint32_t lds_u32(const char* base, uint32_t byte_off) {
    return *reinterpret_cast<const uint32_t*>(base + byte_off);
}

// One 16-index chunk against the lane's fp16 x pairs.
__device__ __forceinline__ float chunk_dot2(const char* lds, uint32_t tb, uint32_t w0, uint32_t w1,
                                            uint32_t w2, const uint32_t (&xh)[8]) {
    uint32_t p[8];
    p[0] = lds_u32(lds, pair_addr<0>(w0, w1, w2, tb));
    p[1] = lds_u32(lds, pair_addr<12>(w0, w1, w2, tb));
    p[2] = lds_u32(lds, pair_addr<24>(w0, w1, w2, tb));
    p[3] = lds_u32(lds, pair_addr<36>(w0, w1, w2, tb));
    p[4] = lds_u32(lds, pair_addr<48>(w0, w1, w2, tb));
    p[5] = lds_u32(lds, pair_addr<60>(w0, w1, w2, tb));
    p[6] = lds_u32(lds, pair_addr<72>(w0, w1, w2, tb));
    p[7] = lds_u32(lds, pair_addr<84>(w0, w1, w2, tb));
    float h0 = 0.f, h1 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k += 2) {
        h0 = dot2(p[k], xh[k], h0);
        h1 = dot2(p[k + 1], xh[k + 1], h1);
    }
    return h0 + h1;
}

template <int NI>
__global__ __launch_bounds__(1024) void lut6_tile_kernel(const TileArgs a) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    __shared__ float ssp[16];
    __shared__ float fin[2][32];

    const int C = a.C, P = a.P;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wi = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
    const int mt = wi / P, w = wi - mt * P;       // matrix, wave within the matrix
    const int g = 64 * w + lane;                  // lane index within the matrix's waves
    const int d = g / C, pos = g - d * C;
    const int r0 = blockIdx.x * a.T;              // first row of the tile
    const int grp = r0 >> 5;                      // LUT group
    const bool xl_owner = mt == 0 && g < C;       // loads x for chunk `pos`
    const int n_waves = a.n_mat * P;
    uint32_t* xs = reinterpret_cast<uint32_t*>(lds + a.n_mat * 16384);   // [8][C]

    // 1. small loads first: LUT entries, x chunk, norm weight chunk
    const uint32_t lut0 = a.lut[0][(size_t)grp * 64 + lane];
    const uint32_t lut1 = a.n_mat > 1 ? a.lut[1][(size_t)grp * 64 + lane] : 0u;
    float4 xv[4], nv[4];
    if (xl_owner) {
        const float4* xp = reinterpret_cast<const float4*>(a.x + (size_t)pos * 16);
#pragma unroll
        for (int q = 0; q < 4; q++) xv[q] = xp[q];
        if (a.nw) {
            const float4* np = reinterpret_cast<const float4*>(a.nw + (size_t)pos * 16);
#pragma unroll
            for (int q = 0; q < 4; q++) nv[q] = np[q];
        }
    }
    // 2. the weight stream of this lane
    // (select, not a.w[mt]: a runtime index into the argument struct becomes a
    // vector load whose wait would also wait for the x loads above)
    // Raw buffer loads over the tile (bounds-checked by the descriptor): the
    // base stays in scalar registers, the lane offset is 32-bit, and the
    // per-instruction step is a scalar offset.
    const uint8_t* Wt = (mt ? a.w[1] : a.w[0]) + (size_t)r0 * C * 12;
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void*)Wt, 0, a.T * C * 12, kBufferRsrcWord3);
    const int voff = (w * 64 + lane) * 12;
    u32x3 wv[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) wv[m] = __builtin_amdgcn_raw_buffer_load_b96(rsrc, voff, m * P * 768, 0);
    // 3. pair tables: wave wi writes rows i1 = wi, wi + n_waves, ... of both
    for (int ri = wi; ri < a.n_mat * 64; ri += n_waves) {
        const int tm = ri >> 6, i1 = ri & 63;
        const uint32_t mine = tm ? lut1 : lut0;
        const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)mine, i1);
        *reinterpret_cast<uint32_t*>(lds + tm * 16384 + i1 * 256 + lane * 4) = mine | (hi << 16);
    }
    // 4. RMSNorm statistics over x (each position is owned once)
    float ss = 0.f;
    if (xl_owner && a.nw) {
#pragma unroll
        for (int q = 0; q < 4; q++)
            ss += xv[q].x * xv[q].x + xv[q].y * xv[q].y + xv[q].z * xv[q].z + xv[q].w * xv[q].w;
    }
    if (a.nw && mt == 0) {
        ss = wave_sum(ss);
        if (lane == 0) ssp[w] = ss;
    }
    __syncthreads();
    if (xl_owner) {
        float xf[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            xf[4 * q] = xv[q].x; xf[4 * q + 1] = xv[q].y; xf[4 * q + 2] = xv[q].z; xf[4 * q + 3] = xv[q].w;
        }
        if (a.nw) {
            float tot = 0.f;
            for (int i = 0; i < P; i++) tot += ssp[i];
            const float inv = 1.0f / sqrtf(tot / (float)a.in_dim + a.eps);
            float nf[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                nf[4 * q] = nv[q].x; nf[4 * q + 1] = nv[q].y; nf[4 * q + 2] = nv[q].z; nf[4 * q + 3] = nv[q].w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) xf[i] = (xf[i] * inv) * nf[i];
        }
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const _Float16 h0 = (_Float16)xf[2 * k], h1 = (_Float16)xf[2 * k + 1];
            xs[k * C + pos] = __builtin_bit_cast(uint32_t, half2_t{h0, h1});
        }
    }
    __syncthreads();
    uint32_t xh[8];
#pragma unroll
    for (int k = 0; k < 8; k++) xh[k] = xs[k * C + pos];
    // 5. dot products
    const uint32_t tb = (uint32_t)mt * 16384u;
    float part[NI];
#pragma unroll
    for (int m = 0; m < NI; m++) part[m] = chunk_dot2(lds, tb, wv[m].x, wv[m].y, wv[m].z, xh);
    // 6. row sums: partials [mt][m][g] in LDS (over the dead tables), then
    // tpr threads per row sum the C partials of the row in a fixed order.
    __syncthreads();
    float* red = reinterpret_cast<float*>(lds);
    const int stride = 64 * P;
#pragma unroll
    for (int m = 0; m < NI; m++) red[(mt * NI + m) * stride + g] = part[m];
    __syncthreads();
    {
        const int tpr = a.tpr, T = a.T;
        const int grp_t = tid / tpr, j = tid - grp_t * tpr;
        float s = 0.f;
        const bool active = grp_t < a.n_mat * T;
        int rm = 0, rr = 0;
        if (active) {
            rm = grp_t / T;
            rr = grp_t - rm * T;
            const int m = rr / a.RP, dd = rr - m * a.RP;
            const float* src = red + (rm * NI + m) * stride + C * dd;
            for (int i = j; i < C; i += tpr) s += src[i];
        }
        for (int msk = tpr >> 1; msk >= 1; msk >>= 1) s += __shfl_xor(s, msk, 64);
        if (active && j == 0) fin[rm][rr] = s;
    }
    __syncthreads();
    if (tid < a.T) {
        const int r = r0 + tid;
        if (a.mode == kOutH) {
            const float gv = fin[0][tid];
            a.y[0][r] = (gv / (1.0f + expf(-gv))) * fin[1][tid];
        } else if (a.mode == kOutGU) {
            a.y[0][r] = fin[0][tid];
            a.y[1][r] = fin[1][tid];
        } else {
            a.y[0][r] = a.residual ? a.y[0][r] + fin[0][tid] : fin[0][tid];
        }
    }
}

// Tile geometry for in_dim, or false when the fast path does not apply.
struct TileGeom {
    int C, P, RP;
};
bool tile_geom(int in_dim, int n_mat, TileGeom& g) {
    if (in_dim % 32 != 0) return false;
    const int C = in_dim / 16;
    int gc = 64;
    while (C % gc) gc >>= 1;
    const int P = C / gc;
    if (P * n_mat > 16) return false;
    g.C = C;
    g.P = P;
    g.RP = 64 / gc;
    return g.RP <= 32;
}

// Launches the tile kernel with about `want_ni` instructions per wave (rows
// per tile = NI * RP, at most 32 so a tile stays in one LUT group).
int tile_launch(TileArgs a, const TileGeom& g, int out_dim, int want_ni, hipStream_t st) {
    a.C = g.C;
    a.P = g.P;
    a.RP = g.RP;
    int ni = want_ni;
    while (ni > 1 && ni * g.RP > 32) ni >>= 1;
    a.T = ni * g.RP;
    const int nt = a.n_mat * g.P * 64;
    int tpr = 64;
    while (tpr > 1 && a.n_mat * a.T * tpr > nt) tpr >>= 1;
    a.tpr = tpr;
    const size_t tabs = (size_t)a.n_mat * 16384 + (size_t)g.C * 32;
    const size_t red = (size_t)a.n_mat * ni * g.P * 64 * 4;
    const size_t lds = tabs > red ? tabs : red;
    const dim3 grid(out_dim / a.T), block(nt);
    switch (ni) {
        case 1: hipLaunchKernelGGL(lut6_tile_kernel<1>, grid, block, lds, st, a); break;
        case 2: hipLaunchKernelGGL(lut6_tile_kernel<2>, grid, block, lds, st, a); break;
        case 4: hipLaunchKernelGGL(lut6_tile_kernel<4>, grid, block, lds, st, a); break;
        case 8: hipLaunchKernelGGL(lut6_tile_kernel<8>, grid, block, lds, st, a); break;
        default: hipLaunchKernelGGL(lut6_tile_kernel<16>, grid, block, lds, st, a); break;
    }
    ANELM_LAUNCHED("lut6_tile_kernel");
    return ANELM_OK;
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

// h = silu(g) * u (qwen3_5.cpp:1123-1126)
__global__ void swiglu_kernel(float* h, const float* g, const float* u, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) {
        const float gv = g[i];
        h[i] = (gv / (1.0f + expf(-gv))) * u[i];
    }
}

// h[r][i] = silu(gu[r][i]) * gu[r][n + i]: the gate and up projections of row r
// computed as one projection with 2n outputs (gate rows first).  Row r is
// blockIdx.y; each thread takes 4 consecutive elements (float4 when n % 4 == 0).
__global__ void swiglu_rows_kernel(float* h, const float* gu, int n) {
    const int r = blockIdx.y, i0 = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    const float* g = gu + (size_t)r * 2 * n;
    float* hr = h + (size_t)r * n;
    if ((n & 3) == 0) {
        if (i0 < n) {
            const float4 gv = *reinterpret_cast<const float4*>(g + i0);
            const float4 uv = *reinterpret_cast<const float4*>(g + n + i0);
            float4 o;
            o.x = (gv.x / (1.0f + expf(-gv.x))) * uv.x;
            o.y = (gv.y / (1.0f + expf(-gv.y))) * uv.y;
            o.z = (gv.z / (1.0f + expf(-gv.z))) * uv.z;
            o.w = (gv.w / (1.0f + expf(-gv.w))) * uv.w;
            *reinterpret_cast<float4*>(hr + i0) = o;
        }
        return;
    }
    for (int i = i0; i < min(i0 + 4, n); i++) {
        const float gv = g[i];
        hr[i] = (gv / (1.0f + expf(-gv))) * g[n + i];
    }
}

// ---------------------------------------------------------------- top-k
// Ordering (value desc, index asc): a precedes b.
__device__ __forceinline__ bool before(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

constexpr int kTopkChunk = 8192;   // logits per selection workgroup (4 waves x 2048)

// Wave-resident selection: lane i holds the i-th best (value, index) of the
// wave's list, best first under `before`; lanes past the list hold (-inf, max).
struct Cand {
    float v;
    int i;
};
__device__ __forceinline__ Cand xchg(Cand c, int mask) {
    return Cand{__shfl_xor(c.v, mask, 64), __shfl_xor(c.i, mask, 64)};
}
// One compare-exchange stage of a bitonic network over the 64 lanes: lanes
// lane and lane ^ stride form a pair; in blocks where (lane & size) == 0 the
// better element goes to the lower lane, in the others to the upper one.
__device__ __forceinline__ Cand bitonic_step(Cand c, int lane, int size, int stride) {
    const Cand p = xchg(c, stride);
    const bool lower = (lane & stride) == 0;
    const bool desc = (lane & size) == 0;
    const bool mine = before(c.v, c.i, p.v, p.i);
    return (lower == desc) == mine ? c : p;
}
// Sorts the 64 lanes' candidates best first.
__device__ __forceinline__ Cand wave_sort(Cand c, int lane) {
#pragma unroll
    for (int size = 2; size <= 64; size <<= 1)
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) c = bitonic_step(c, lane, size, stride);
    return c;
}
// Top 64 of two lists sorted best first: the lane-wise better of L[i] and
// N[63 - i] is bitonic; a half-cleaner cascade sorts it.
__device__ __forceinline__ Cand wave_merge(Cand L, Cand N, int lane) {
    const Cand r = Cand{__shfl(N.v, 63 - lane, 64), __shfl(N.i, 63 - lane, 64)};
    Cand c = before(L.v, L.i, r.v, r.i) ? L : r;
#pragma unroll
    for (int stride = 32; stride > 0; stride >>= 1) c = bitonic_step(c, lane, 64, stride);
    return c;
}
// Adds 64 unsorted candidates (one per lane) to the list L holding the best k;
// skipped when none beats the list's k-th entry.
__device__ __forceinline__ Cand wave_offer(Cand L, Cand c, int lane, int k) {
    const float tv = __shfl(L.v, k - 1, 64);
    const int ti = __shfl(L.i, k - 1, 64);
    if (!__any(before(c.v, c.i, tv, ti))) return L;
    return wave_merge(L, wave_sort(c, lane), lane);
}

// Stage 1: each workgroup selects the best k of one chunk of one batch row's
// logits -- every wave selects over its quarter, then wave 0 merges the four
// lists -- into candidates [batch][n_chunks][k].
//
// A wave first loads its 2048 logits (32 per lane) and sorts the 64 lane
// maxima once; the k-th best lane maximum T is a threshold: the k lanes whose
// maxima are not after T supply k elements that precede every element after
// T, so the best k lie among the elements not after T.  Only those are queued
// (64 LDS slots per wave, compacted by ballot prefix) and offered to the
// running list when the queue fills and at the end; on random logits that is
// one or two sort-and-merge passes per wave instead of 32.  The result is the
// same (value desc, index asc) list as offering every element.
constexpr int kTopkPerLane = kTopkChunk / 4 / 64;
__global__ __launch_bounds__(256) void topk_stage1(const float* logits, int n, int k, int n_chunks,
                                                   float* cv, int* ci) {
    __shared__ Cand lists[4][64];
    __shared__ Cand queue[4][64];
    const int chunk = blockIdx.x, b = blockIdx.y;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const float* row = logits + (size_t)b * n;
    const int base = chunk * kTopkChunk + w * (kTopkChunk / 4);
    float v[kTopkPerLane];
#pragma unroll
    for (int t = 0; t < kTopkPerLane; t++) v[t] = row[min(base + t * 64 + lane, n - 1)];
    auto idx_of = [&](int t) { return base + t * 64 + lane < n ? base + t * 64 + lane : 0x7fffffff; };
    Cand m{-INFINITY, 0x7fffffff};
#pragma unroll
    for (int t = 0; t < kTopkPerLane; t++) {
        const int it = idx_of(t);
        // a NaN logit ranks as -inf (keeping its index for ties), so the
        // ordering stays total and NaN never wins the greedy pick
        const float vt = (it != 0x7fffffff && !__builtin_isnan(v[t])) ? v[t] : -INFINITY;
        v[t] = vt;
        if (before(vt, it, m.v, m.i)) m = Cand{vt, it};
    }
    const Cand sm = wave_sort(m, lane);
    const float tv = __shfl(sm.v, k - 1, 64);
    const int ti = __shfl(sm.i, k - 1, 64);

    Cand L{-INFINITY, 0x7fffffff};
    int filled = 0;   // queue entries in use (wave-uniform)
#pragma unroll
    for (int t = 0; t < kTopkPerLane; t++) {
        const int it = idx_of(t);
        const bool pass = !before(tv, ti, v[t], it);
        const uint64_t bits = __ballot(pass);
        const int cnt = __popcll(bits);
        if (cnt == 0) continue;
        if (filled + cnt > 64) {
            __builtin_amdgcn_wave_barrier();
            const Cand q = lane < filled ? queue[w][lane] : Cand{-INFINITY, 0x7fffffff};
            __builtin_amdgcn_wave_barrier();
            L = wave_offer(L, q, lane, k);
            filled = 0;
        }
        if (pass) {
            const int pos = filled + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bits >> 32),
                                                                     __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0u));
            queue[w][pos] = Cand{v[t], it};
        }
        filled += cnt;
    }
    __builtin_amdgcn_wave_barrier();
    const Cand q = lane < filled ? queue[w][lane] : Cand{-INFINITY, 0x7fffffff};
    L = wave_offer(L, q, lane, k);

    lists[w][lane] = L;
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int o = 1; o < 4; o++) L = wave_merge(L, lists[o][lane], lane);
    if (lane < k) {
        cv[((size_t)b * n_chunks + chunk) * k + lane] = L.v;
        ci[((size_t)b * n_chunks + chunk) * k + lane] = L.i;
    }
}

// Stage 2: one workgroup per batch row merges the row's chunk candidates:
// wave w takes lists w*8 .. w*8+7, then w+32 .., loading eight at once, and
// wave 0 merges the four lists.  Entries are distinct under (value desc,
// index asc), so the merge order does not change the result.
constexpr int kTopkGroup = 8;
__global__ __launch_bounds__(256) void topk_stage2(const float* cv, const int* ci, int n_chunks, int k,
                                                   int32_t* out_idx, float* out_val) {
    __shared__ Cand lists[4][64];
    const int b = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int le = min(lane, k - 1);
    Cand L{-INFINITY, 0x7fffffff};
    for (int c0 = w * kTopkGroup; c0 < n_chunks; c0 += 4 * kTopkGroup) {
        Cand cur[kTopkGroup];
#pragma unroll
        for (int g = 0; g < kTopkGroup; g++) {
            const size_t o = ((size_t)b * n_chunks + min(c0 + g, n_chunks - 1)) * k + le;
            cur[g] = Cand{cv[o], ci[o]};
        }
#pragma unroll
        for (int g = 0; g < kTopkGroup; g++) {
            // lists past n_chunks and lanes past k are empty entries; the lists
            // arrive sorted
            const bool ok = c0 + g < n_chunks && lane < k;
            L = wave_merge(L, ok ? cur[g] : Cand{-INFINITY, 0x7fffffff}, lane);
        }
    }
    lists[w][lane] = L;
    __syncthreads();
    if (w != 0) return;
#pragma unroll
    for (int o = 1; o < 4; o++) L = wave_merge(L, lists[o][lane], lane);
    if (lane < k) {
        out_idx[(size_t)b * k + lane] = L.i;
        out_val[(size_t)b * k + lane] = L.v;
    }
}

constexpr int kMaxNJ = 11;   // in_dim up to 11264: pair table 16 KiB + x 44 KiB of LDS

// Rows per wave: 4 while the lane's x chunks are few; 2 for wide inputs so the
// register footprint (x + weights in flight) keeps two waves per SIMD.
template <int NJ>
constexpr int rows_per_wave() { return NJ <= 4 ? 4 : 2; }

template <int NJ, int STAGE>
int gemv_launch(GemvArgs a, int n_mats, hipStream_t st) {
    constexpr int RPW = rows_per_wave<NJ>();
    const int rows_per_block = kNW * RPW;
    const int blocks = a.out_dim / rows_per_block;
    a.blocks0 = blocks;
    const size_t lds = (size_t)kPairs * sizeof(uint32_t) + (size_t)a.in_dim * sizeof(float);
    hipLaunchKernelGGL((lut6_gemv_kernel<NJ, RPW, STAGE>), dim3(blocks * n_mats), dim3(kNT), lds, st, a);
    ANELM_LAUNCHED("lut6_gemv_kernel");
    return ANELM_OK;
}

template <int STAGE>
int gemv_dispatch(GemvArgs a, int n_mats, hipStream_t st) {
    const int nj = (a.in_dim / 16 + 63) / 64;
    switch (nj) {
#define CASE(N) case N: return gemv_launch<N, STAGE>(a, n_mats, st);
        CASE(1) CASE(2) CASE(3) CASE(4) CASE(5) CASE(6) CASE(7) CASE(8) CASE(9) CASE(10) CASE(11)
#undef CASE
        default: return set_error(ANELM_ERANGE, "lut6: in_dim %d beyond %d", a.in_dim, kMaxNJ * 1024);
    }
}

int check_shape(int out_dim, int in_dim) {
    ANELM_REQUIRE(out_dim > 0 && out_dim % 32 == 0, "lut6: out_dim %d must be a positive multiple of 32", out_dim);
    ANELM_REQUIRE(in_dim > 0 && in_dim % 16 == 0, "lut6: in_dim %d must be a positive multiple of 16", in_dim);
    ANELM_REQUIRE(in_dim <= kMaxNJ * 1024, "lut6: in_dim %d beyond %d", in_dim, kMaxNJ * 1024);
    return ANELM_OK;
}

// g = gate n, u = up n with n = rmsnorm(x) (or x); with h != NULL the SwiGLU
// product h = silu(g) * u is written instead.  Only the fallback path stores
// g and u then: into the given buffers (h may alias g), else the workspace.
int gate_up(float* g, float* u, float* h, const float* x, const float* norm_w, float eps,
            const uint8_t* gw, const uint16_t* gl, const uint8_t* uw, const uint16_t* ul, int hidden,
            int inter, hipStream_t st) {
    TileGeom geo;
    if (tile_geom(hidden, 2, geo)) {
        TileArgs a{};
        a.w[0] = gw;
        a.lut[0] = gl;
        a.w[1] = uw;
        a.lut[1] = ul;
        a.y[0] = h ? h : g;
        a.y[1] = h ? nullptr : u;
        a.x = x;
        a.nw = norm_w;
        a.eps = eps;
        a.n_mat = 2;
        a.mode = h ? kOutH : kOutGU;
        a.in_dim = hidden;
        return tile_launch(a, geo, inter, 8, st);
    }
    if (h && !(g && u)) {
        float* gu = static_cast<float*>(workspace((size_t)2 * inter * sizeof(float), st));
        if (!gu) return ANELM_ENOMEM;
        g = gu;
        u = gu + inter;
    }
    GemvArgs a{};
    a.w[0] = gw;
    a.lut[0] = gl;
    a.y[0] = g;
    a.w[1] = uw;
    a.lut[1] = ul;
    a.y[1] = u;
    a.out_dim = inter;
    a.in_dim = hidden;
    a.x = x;
    a.nw = norm_w;
    a.eps = eps;
    int rc = norm_w ? gemv_dispatch<kStageNorm>(a, 2, st) : gemv_dispatch<kStageCopy>(a, 2, st);
    if (rc || !h) return rc;
    hipLaunchKernelGGL(swiglu_kernel, dim3((inter + 255) / 256), dim3(256), 0, st, h, g, u, inter);
    ANELM_LAUNCHED("swiglu_kernel");
    return ANELM_OK;
}

// y = W x, or y += W x with `residual`; with norm_w, x is first replaced by
// rmsnorm(x, norm_w, eps) (cpu_ops.cpp:24-30).
int gemv(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int out_dim, int in_dim,
         int residual, hipStream_t st, const float* norm_w = nullptr, float eps = 0.f) {
    TileGeom geo;
    if (tile_geom(in_dim, 1, geo)) {
        TileArgs a{};
        a.w[0] = w;
        a.lut[0] = lut;
        a.y[0] = y;
        a.x = x;
        a.nw = norm_w;
        a.eps = eps;
        a.n_mat = 1;
        a.mode = kOutY;
        a.residual = residual;
        a.in_dim = in_dim;
        // long rows (in_dim >= 3072: the down projections) take tiles of 4
        // instructions per wave: the per-tile set-up is small beside a row
        // there, and the smaller tiles spread over the compute units more
        // evenly (9216 -> 2560: 10.2 -> 9.3 us; 3584 -> 1024: 5.7 -> 4.6 us)
        return tile_launch(a, geo, out_dim, in_dim >= 3072 ? 4 : 8, st);
    }
    GemvArgs a{};
    a.w[0] = w;
    a.lut[0] = lut;
    a.y[0] = y;
    a.out_dim = out_dim;
    a.in_dim = in_dim;
    a.x = x;
    a.nw = norm_w;
    a.eps = eps;
    a.residual = residual;
    return norm_w ? gemv_dispatch<kStageNorm>(a, 1, st) : gemv_dispatch<kStageCopy>(a, 1, st);
}

// Y[b] (+)= W X[b] for b < batch: the MFMA GEMM over tiles of 32 inputs.  The
// columns are cut into S equal slices (each a valid register-resident window,
// a multiple of 256 columns when S > 1): S is the smallest count that fits,
// raised until the (32-row group, slice) units cover every CU twice, so small
// projections still fill the chip.  With S > 1 one launch writes the slices'
// partial products (second workspace) and split_sum adds them (and Y when
// accumulating) -- a fixed order, so results do not vary between calls.
// Shapes that fit no slicing take one GEMV per input.
int batched_gemv(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int batch, int out_dim,
                 int in_dim, int accumulate, hipStream_t st, const float* norm_w = nullptr, float eps = 0.f,
                 float* xn = nullptr) {
    // with norm_w: xn = RMSNorm(y) * norm_w per row afterwards
    auto norm_rows = [&](int b0, int nb) {
        return anelm_rmsnorm(xn + (size_t)b0 * out_dim, y + (size_t)b0 * out_dim, norm_w, out_dim, nb, out_dim,
                             out_dim, eps, st);
    };
    int np = 0, waves = 0;
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 15) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    auto fits = [&](int s) {
        return in_dim % s == 0 && lut6_gemm_geometry(in_dim / s, np, waves) && (s == 1 || (in_dim / s) % 256 == 0);
    };
    int ns = 1;
    while (ns <= 64 && !fits(ns)) ns++;
    if (!aligned || ns > 64) {
        for (int b = 0; b < batch; b++) {
            const int rc = gemv(y + (size_t)b * out_dim, w, lut, x + (size_t)b * in_dim, out_dim, in_dim, accumulate, st);
            if (rc) return rc;
        }
        return norm_w ? norm_rows(0, batch) : ANELM_OK;
    }
    Device* dev = device();
    if (!dev) return ANELM_EHIP;
    const int n_groups = out_dim / 32;
    for (int s = ns + 1; n_groups * ns < 2 * dev->num_cus && s <= 64; s++)
        if (fits(s)) ns = s;
    if (!fits(ns)) return set_error(ANELM_EINVAL, "lut6_gemm: no column split for in_dim %d", in_dim);
    const int part = in_dim / ns;
    const long ldw = (long)in_dim * 3 / 4;
    for (int b0 = 0; b0 < batch; b0 += 32) {
        const int nb = batch - b0 < 32 ? batch - b0 : 32;
        float* yb = y + (size_t)b0 * out_dim;
        const float* xb = x + (size_t)b0 * in_dim;
        if (ns == 1) {
            int rc = lut6_gemm_launch(yb, w, ldw, lut, xb, in_dim, nb, out_dim, part, accumulate, 1, 0, st);
            if (rc == ANELM_OK && norm_w) rc = norm_rows(b0, nb);
            if (rc) return rc;
            continue;
        }
        const long n = (long)nb * out_dim;
        float* parts = static_cast<float*>(workspace2((size_t)ns * n * sizeof(float), st));
        if (!parts) return ANELM_ENOMEM;
        int rc = lut6_gemm_launch(parts, w, ldw, lut, xb, in_dim, nb, out_dim, part, 0, ns, n, st);
        if (rc) return rc;
        if (norm_w && lut6_split_sum_norm_fits(out_dim, ns)) {
            rc = lut6_split_sum_norm(yb, parts, n, ns, accumulate, nb, out_dim, norm_w, eps,
                                     xn + (size_t)b0 * out_dim, st);
        } else {
            rc = lut6_split_sum(yb, parts, n, ns, accumulate, st);
            if (rc == ANELM_OK && norm_w) rc = norm_rows(b0, nb);
        }
        if (rc) return rc;
    }
    return ANELM_OK;
}

}  // namespace
}  // namespace anelm

using namespace anelm;

namespace anelm {
int lut6_gemv_impl(float* y, const uint8_t* w, const uint16_t* lut, const float* x, const float* norm_w,
                   float eps, int out_dim, int in_dim, int residual, hipStream_t st) {
    int rc = check_shape(out_dim, in_dim);
    if (rc) return rc;
    return gemv(y, w, lut, x, out_dim, in_dim, residual, st, norm_w, eps);
}
}  // namespace anelm

namespace anelm {
int lut6_gemm_norm(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int batch, int out_dim,
                   int in_dim, int accumulate, const float* norm_w, float eps, float* xn, hipStream_t st) {
    ANELM_NONNULL(norm_w);
    ANELM_NONNULL(xn);
    int rc = check_shape(out_dim, in_dim);
    if (rc) return rc;
    ANELM_REQUIRE(batch > 0, "lut6_gemm: batch %d", batch);
    return batched_gemv(y, w, lut, x, batch, out_dim, in_dim, accumulate, st, norm_w, eps, xn);
}
}  // namespace anelm

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
    return gemv(y, w, lut, x, out_dim, in_dim, 0, as_stream(stream));
}

int anelm_lut6_proj(float* y, const uint8_t* w, const uint16_t* lut, const float* x, const float* norm_w,
                    float eps, int out_dim, int in_dim, int accumulate, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(w);
    ANELM_NONNULL(lut);
    ANELM_NONNULL(x);
    ANELM_REQUIRE(accumulate == 0 || accumulate == 1, "lut6_proj: accumulate %d", accumulate);
    ANELM_REQUIRE(!(accumulate && norm_w && y == x), "lut6_proj: y aliases the normalised input");
    return lut6_gemv_impl(y, w, lut, x, norm_w, eps, out_dim, in_dim, accumulate, as_stream(stream));
}

int anelm_lut6_gate_up(float* g, float* u, const float* x, const float* norm_w, float eps,
                       const uint8_t* gate_w, const uint16_t* gate_lut, const uint8_t* up_w,
                       const uint16_t* up_lut, int hidden, int inter, void* stream) {
    ANELM_NONNULL(g);
    ANELM_NONNULL(u);
    ANELM_NONNULL(x);
    ANELM_NONNULL(gate_w);
    ANELM_NONNULL(gate_lut);
    ANELM_NONNULL(up_w);
    ANELM_NONNULL(up_lut);
    int rc = check_shape(inter, hidden);
    if (rc) return rc;
    return gate_up(g, u, nullptr, x, norm_w, eps, gate_w, gate_lut, up_w, up_lut, hidden, inter,
                   as_stream(stream));
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
    return gate_up(nullptr, nullptr, h, x, norm_w, eps, gate_w, gate_lut, up_w, up_lut, hidden, inter,
                   as_stream(stream));
}

int anelm_lut6_ffn(float* x, float* gu_scratch, const float* norm_w, float eps,
                   const uint8_t* gate_w, const uint16_t* gate_lut, const uint8_t* up_w,
                   const uint16_t* up_lut, const uint8_t* down_w, const uint16_t* down_lut,
                   int hidden, int inter, void* stream) {
    ANELM_NONNULL(x);
    ANELM_NONNULL(gu_scratch);
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
    float* h = gu_scratch;
    rc = gate_up(gu_scratch, gu_scratch + inter, h, x, norm_w, eps, gate_w, gate_lut, up_w, up_lut,
                 hidden, inter, st);
    if (rc) return rc;
    return gemv(x, down_w, down_lut, h, hidden, inter, 1, st);
}

int anelm_lut6_gemm(float* y, const uint8_t* w, const uint16_t* lut, const float* x, int batch, int out_dim,
                    int in_dim, int accumulate, void* stream) {
    ANELM_NONNULL(y);
    ANELM_NONNULL(w);
    ANELM_NONNULL(lut);
    ANELM_NONNULL(x);
    int rc = check_shape(out_dim, in_dim);
    if (rc) return rc;
    ANELM_REQUIRE(batch > 0, "lut6_gemm: batch %d", batch);
    ANELM_REQUIRE(accumulate == 0 || accumulate == 1, "lut6_gemm: accumulate %d", accumulate);
    return batched_gemv(y, w, lut, x, batch, out_dim, in_dim, accumulate, as_stream(stream));
}

int anelm_swiglu(float* h, const float* g, const float* u, int64_t n, void* stream) {
    ANELM_NONNULL(h);
    ANELM_NONNULL(g);
    ANELM_NONNULL(u);
    ANELM_REQUIRE(n >= 0 && n <= 0x7fffffffLL - 255, "swiglu: n %lld", (long long)n);
    if (n == 0) return ANELM_OK;
    hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), h, g, u,
                       (int)n);
    ANELM_LAUNCHED("swiglu_kernel");
    return ANELM_OK;
}

int anelm_swiglu_rows(float* h, const float* gu, int rows, int n, void* stream) {
    ANELM_NONNULL(h);
    ANELM_NONNULL(gu);
    ANELM_REQUIRE(rows >= 0 && n >= 0, "swiglu_rows: rows %d n %d", rows, n);
    ANELM_REQUIRE(rows <= 65535, "swiglu_rows: rows %d (at most 65535)", rows);
    if (rows == 0 || n == 0) return ANELM_OK;
    // 16-byte rows need 16-byte aligned buffers for the float4 path
    ANELM_REQUIRE((n & 3) != 0 || ((reinterpret_cast<uintptr_t>(h) | reinterpret_cast<uintptr_t>(gu)) & 15) == 0,
                  "swiglu_rows: buffers must be 16-byte aligned");
    hipLaunchKernelGGL(swiglu_rows_kernel, dim3((unsigned)((n + 1023) / 1024), (unsigned)rows), dim3(256), 0,
                       as_stream(stream), h, gu, n);
    ANELM_LAUNCHED("swiglu_rows_kernel");
    return ANELM_OK;
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
    ANELM_REQUIRE(batch > 0 && batch <= 65535, "lut6_topk: batch %d (1..65535)", batch);
    ANELM_REQUIRE(k > 0 && k <= 64 && k <= out_dim, "lut6_topk: k %d must be in [1, min(64, out_dim)]", k);
    hipStream_t st = as_stream(stream);
    const int n_chunks = (out_dim + kTopkChunk - 1) / kTopkChunk;
    const int n_cand = n_chunks * k;
    const size_t logits_bytes = (size_t)batch * out_dim * sizeof(float);
    const size_t cand_bytes = (size_t)batch * n_cand * (sizeof(float) + sizeof(int));
    char* ws = static_cast<char*>(workspace(logits_bytes + cand_bytes, st));
    if (!ws) return ANELM_ENOMEM;
    float* logits = reinterpret_cast<float*>(ws);
    float* cv = reinterpret_cast<float*>(ws + logits_bytes);
    int* ci = reinterpret_cast<int*>(ws + logits_bytes + (size_t)batch * n_cand * sizeof(float));
    rc = batched_gemv(logits, w, lut, x, batch, out_dim, in_dim, 0, st);
    if (rc) return rc;
    hipLaunchKernelGGL(topk_stage1, dim3(n_chunks, batch), dim3(256), 0, st, logits, out_dim, k,
                       n_chunks, cv, ci);
    ANELM_LAUNCHED("topk_stage1");
    hipLaunchKernelGGL(topk_stage2, dim3(batch), dim3(256), 0, st, cv, ci, n_chunks, k, out_idx, out_val);
    ANELM_LAUNCHED("topk_stage2");
    return ANELM_OK;
}

}  // extern "C"
