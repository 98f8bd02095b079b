// Batched LUT6 GEMM on fp16 MFMA: Y[b][r] = sum_c W[r][c] * X[b][c] for up to
// 32 input vectors at once, each 32-row LUT group of W decoded ONCE for all of
// them.  Used by the LM head (top-k over the logits of a batch of hidden
// states, scripts/export_hybrid_chunks.py:409-421) and by batched LUT6
// projections; a batch of one goes through the same path.
//
// Mapping (v_mfma_f32_32x32x16_f16, A = 32 weight rows x 16 columns, B = 16
// columns x 32 batch vectors, C = 32 rows x 32 vectors):
//   * a workgroup walks 32-row groups g (one LUT per group); its NW waves split
//     the columns: wave w owns the window [w*128*NP, (w+1)*128*NP);
//   * lane l = (m, hh), m = l % 32, hh = l / 32, feeds weight row m and batch
//     vector m; MFMA step t of the wave contracts columns
//     w*128*NP + hh*64*NP + 8t + j (j < 8).  The contraction order over the
//     columns is permuted identically in A and B, so each lane's weights are
//     one contiguous 48*NP-byte stretch of its row;
//   * the wave's X window sits in registers for the whole launch (fp16, as the
//     LUT6 path takes its activations); a group's weights are staged in LDS
//     one group ahead by coalesced loads (1 KiB per wave instruction) and
//     taken into registers from there; each 12-bit field (two indices) dequantises
//     through a 4096-entry pair table T[(i1 << 6) | i0] = (lut[i0], lut[i1])
//     built per group in LDS (double-buffered);
//   * the NW partial 32x32 tiles are summed through LDS and written as fp32.
// Reference math: matvec (core/cpu_ops.cpp:77-80) on the dequantised weights.
#include "anelm_internal.hpp"

#include <algorithm>

namespace anelm {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTabBytes = 4096 * 4;
constexpr int kLutSlots = 64;                          // LUTs staged per round
constexpr int kLutOff = 2 * kTabBytes;                 // staged LUTs [kLutSlots][64] u16
constexpr int kRedOff = kLutOff + kLutSlots * 128;     // partial tiles [NW][16][kRedRow] f32
// Partial-tile row: lane l of accumulator e sits at (l % 32) + 33 * (l / 32)
// of a 66-float row, so the reduction's reads (32 threads of one vector n:
// all 16 e x 2 half-waves) fall on 32 distinct banks, and so do the writes.
constexpr int kRedRow = 66;
__device__ __forceinline__ int red_pos(int e, int l) { return e * kRedRow + (l & 31) + 33 * (l >> 5); }

struct GemmArgs {
    float* y;              // [batch][out_dim]
    const uint8_t* w;      // row r at w + r * ldw bytes, in_dim * 3 / 4 bytes used
    const uint16_t* lut;   // [out_dim / 32][64]
    const float* x;        // vector b at x + b * ldx, in_dim floats used
    int batch, out_dim, in_dim;
    long ldw, ldx;         // row strides (bytes of w, floats of x): a column slice of wider matrices
    int accumulate;        // y += W x instead of y = W x
    long sw, sx, sy;       // per column slice blockIdx.y: offsets of w (bytes), x and y (floats)
};

// Pair-table byte offset of pair p (indices 2p, 2p + 1: the 12-bit field at
// bit 12p of the lane's weight words), OR-ed with the table base tb.  p is a
// compile-time constant after unrolling, so the shifts and word picks fold.
template <int NWD>
__device__ __forceinline__ uint32_t pair_off(const uint32_t (&wd)[NWD], int p, uint32_t tb) {
    const int s = 12 * p - 2;                  // field lands at bit 2 (4 bytes per entry)
    uint32_t v;
    if (s < 0) {
        v = wd[0] << 2;
    } else {
        const int d = s >> 5, sh = s & 31;
        if (sh + 14 <= 32 || d + 1 >= NWD) v = wd[d] >> sh;
        else v = __builtin_amdgcn_alignbit(wd[d + 1], wd[d], sh);
    }
    return (v & 0x3FFCu) | tb;
}

// Group g's 32 weight rows are staged in LDS before each lane takes its own
// stretch: a lane's operand stretch (48*NP bytes of its row) is 16-byte
// pieces of 32 different rows, which as direct loads touch 64 partial cache
// lines per wave instruction.  Staged, every wave instruction reads 1 KiB of
// consecutive memory.  Row r of the group sits at r * (CH * 16) in the stage,
// CH = row bytes / 16 + 1: the last 16 bytes of a row are padding (loaded
// from past the buffer's end, so zeros), which keeps one wave instruction's
// 64 destination chunks consecutive and puts the operand reads of
// consecutive rows on different banks.
template <int NW, int NP>
struct Stage {
    static constexpr int RB = NW * 96 * NP;                // row bytes of this column slice
    static constexpr int CH = RB / 16 + 1;                 // 16-byte chunks per staged row
    static constexpr int NI = (32 * CH + 63) / 64;         // wave instructions per group
    static constexpr int kBytes = NI * 1024;
};
template <int NW, int NP>
__device__ __forceinline__ void stage_group(const GemmArgs& a, int g, char* stage, int w, int lane) {
    using S = Stage<NW, NP>;
    asm volatile("" : "+v"(lane));   // recomputed per group, not held across the loop
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(a.w), 0, (int)((long)a.out_dim * a.ldw), 0x00020000);
    for (int i = w; i < S::NI; i += NW) {
        const int q = i * 64 + lane, row = q / S::CH, c = q - row * S::CH;
        // padding chunks and chunks past the 32 rows read from past the end
        const int off = (row < 32 && c < S::CH - 1) ? (g * 32 + row) * (int)a.ldw + 16 * c : 0x7ffffff0;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)(stage + i * 1024), 16,
                                                 off, 0, 0, 2);
    }
}
// This lane's stretch: row m = lane % 32, bytes w*96*NP + hh*48*NP .. +48*NP.
template <int NW, int NP>
__device__ __forceinline__ void read_group(uint32_t (&wd)[12 * NP], const char* stage, int w, int lane) {
    using S = Stage<NW, NP>;
    asm volatile("" : "+v"(lane));
    const int m = lane & 31, hh = lane >> 5;
    const char* src = stage + m * (S::CH * 16) + w * 96 * NP + hh * 48 * NP;
#pragma unroll
    for (int i = 0; i < 3 * NP; i++) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(src + 16 * i);
        wd[4 * i] = v.x;
        wd[4 * i + 1] = v.y;
        wd[4 * i + 2] = v.z;
        wd[4 * i + 3] = v.w;
    }
}

// Dequantise this lane's 64*NP indices through the pair table at byte offset
// tb and accumulate the wave's 8*NP MFMA steps into c.
template <int NP>
__device__ __forceinline__ void group_mfma(float16_t& c, const uint32_t (&wd)[12 * NP],
                                           const half8 (&xb)[8 * NP], const char* lds, uint32_t tb) {
#pragma unroll
    for (int t = 0; t < 8 * NP; t++) {
        u32x4 av;
        av.x = *reinterpret_cast<const uint32_t*>(lds + pair_off(wd, 4 * t + 0, tb));
        av.y = *reinterpret_cast<const uint32_t*>(lds + pair_off(wd, 4 * t + 1, tb));
        av.z = *reinterpret_cast<const uint32_t*>(lds + pair_off(wd, 4 * t + 2, tb));
        av.w = *reinterpret_cast<const uint32_t*>(lds + pair_off(wd, 4 * t + 3, tb));
        c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8, av), xb[t], c, 0, 0, 0);
    }
}

// Builds the pair table of the workgroup's j-th group (LUT staged in LDS at
// kLutOff) into table `slot`: wave w writes rows i1 = w, w + nw, ... of 64
// entries, lane i0 holding lut[i0].
__device__ __forceinline__ void build_table(char* lds, int slot, int j, int w, int nw, int lane) {
    const uint16_t* l = reinterpret_cast<const uint16_t*>(lds + kLutOff) + (j & (kLutSlots - 1)) * 64;
    uint32_t* tab = reinterpret_cast<uint32_t*>(lds + slot * kTabBytes);
    const uint32_t mine = l[lane];
    for (int i1 = w; i1 < 64; i1 += nw) tab[i1 * 64 + lane] = mine | ((uint32_t)l[i1] << 16);
}

// Stages the LUTs of the workgroup's groups j0 .. j0 + kLutSlots - 1 (group
// index blockIdx.x + j * gridDim.x) that exist into LDS.  Every load is issued
// before the first LDS store (a fixed count per thread), so the staging costs
// one round trip.  Called with every wave between two barriers.
template <int NT>
__device__ __forceinline__ void stage_luts(const GemmArgs& a, char* lds, int j0, int tid) {
    asm volatile("" : "+v"(tid));   // indices recomputed per staging, not held across the group loop
    constexpr int K = (kLutSlots * 64 + NT - 1) / NT;
    uint16_t* l = reinterpret_cast<uint16_t*>(lds + kLutOff);
    const int n_groups = a.out_dim / 32;
    const int mine = (n_groups - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x;   // groups of this workgroup
    const int n_e = min(kLutSlots, mine - j0) * 64;
    uint16_t v[K];
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int e = tid + k * NT;
        const int g = (int)blockIdx.x + (j0 + (e >> 6)) * (int)gridDim.x;
        v[k] = a.lut[(size_t)(e < n_e ? g : (int)blockIdx.x) * 64 + (e & 63)];
    }
#pragma unroll
    for (int k = 0; k < K; k++) {
        const int e = tid + k * NT;
        if (e < n_e) l[e] = v[k];
    }
}

// The wave's X window (vectors n < 32, columns w*128*NP .. +128*NP) as MFMA B
// operands: lane (n, hh) takes columns hh*64*NP + 8t + j.  That is a 128*NP-
// byte stretch of one row per lane, which as direct loads touches 64 partial
// cache lines per wave instruction; instead each wave instruction loads
// consecutive 16-byte chunks of whole rows (1 KiB), converts them to fp16
// into this wave's 4 KiB of LDS (8 rows, RS bytes apart) and each lane takes
// its stretch from there, 8 rows per round.  Vectors past the batch read
// zeros (offsets past the buffer).
template <int NP>
__device__ __forceinline__ void load_x(half8 (&xb)[8 * NP], const GemmArgs& a, char* scratch, int w, int lane) {
    constexpr int C4 = 32 * NP;            // float4 chunks in a row of the window
    constexpr int RS = 256 * NP + 16;      // staged row: 128*NP halves + 16 bytes of bank offset
    constexpr int PER = 8 * C4 / 64;       // chunks per lane per round of 8 rows
    static_assert(8 * RS <= 16 * kRedRow * 4, "x staging exceeds the wave's partial-tile area");
    const uint32_t bytes = (uint32_t)(((long)a.batch - 1) * a.ldx + a.in_dim) * 4u;
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.x), 0, (int)bytes, 0x00020000);
    const int n = lane & 31, hh = lane >> 5;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        u32x4 v[PER];
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = i * 64 + lane, row = 8 * r + q / C4, c4 = q % C4;
            const uint32_t off = row < a.batch ? (uint32_t)(((long)row * a.ldx + w * 128 * NP + 4 * c4) * 4) : bytes;
            v[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, (int)off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < PER; i++) {
            const int q = i * 64 + lane, rl = q / C4, c4 = q % C4;
            typedef _Float16 half4 __attribute__((ext_vector_type(4)));
            // each element copied out before its bit cast (a bit cast of a
            // vector element expression compiles as element 0)
            const uint32_t e0 = v[i].x, e1 = v[i].y, e2 = v[i].z, e3 = v[i].w;
            const half4 hv = {(_Float16)__builtin_bit_cast(float, e0), (_Float16)__builtin_bit_cast(float, e1),
                              (_Float16)__builtin_bit_cast(float, e2), (_Float16)__builtin_bit_cast(float, e3)};
            *reinterpret_cast<half4*>(scratch + rl * RS + c4 * 8) = hv;
        }
        // the wave's own LDS, accessed in order: no barrier
        if ((n >> 3) == r) {
            const char* src = scratch + (n & 7) * RS + hh * 128 * NP;
#pragma unroll
            for (int t = 0; t < 8 * NP; t++) xb[t] = *reinterpret_cast<const half8*>(src + 16 * t);
        }
    }
}

// Sums the NW partial tiles of group g and writes Y[n][32g + m] for n < batch.
// Thread t handles (n = t / 32, m = t % 32): consecutive threads write
// consecutive rows of one output vector.
// The trip count is a compile-time constant, so every thread issues the same
// number of stores per group: the compiler can then count the vector-memory
// events between a weight prefetch and its use (stores count too) and leave
// the prefetch in flight.
// Stores are raw buffer stores over y: an element outside the batch gets an
// offset past the buffer's end, which the hardware drops, so the store is
// issued by every thread without a branch.
template <int NW, bool ACC>
__device__ __forceinline__ void reduce_store(const GemmArgs& a, int g, const char* lds, int tid) {
    constexpr int NT = NW * 64;
    const float* red = reinterpret_cast<const float*>(lds + kRedOff);
    const uint32_t bytes = (uint32_t)a.batch * (uint32_t)a.out_dim * 4u;
    const __amdgpu_buffer_rsrc_t ry = __builtin_amdgcn_make_buffer_rsrc(a.y, 0, (int)bytes, 0x00020000);
#pragma unroll
    for (int k = 0; k < (1024 + NT - 1) / NT; k++) {
        const int t = tid + k * NT;
        const int n = t >> 5, m = t & 31;
        // C layout: accumulator e of lane l holds row 8*(e/4) + 4*(l/32) + e%4, vector l%32
        const int hh = (m >> 2) & 1, e = 4 * (m >> 3) + (m & 3), l = (n & 31) + 32 * hh;
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) s += red[w * 16 * kRedRow + red_pos(e, l)];
        const uint32_t off = (t < 1024 && n < a.batch) ? ((uint32_t)n * (uint32_t)a.out_dim + (uint32_t)g * 32u +
                                                            (uint32_t)m) * 4u
                                                         : bytes;
        if constexpr (ACC)   // out-of-range offsets read 0 and drop the store
            s += __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ry, (int)off, 0, 0));
        __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, s), ry, (int)off, 0, 0);
    }
}

// NP = 2: 64 registers of X per lane; NP = 1: 32.
template <int NP, int NW, bool ACC>
__global__ __launch_bounds__(NW * 64) void lut6_gemm_kernel(const GemmArgs a0) {
    extern __shared__ __attribute__((aligned(16))) char lds[];
    // column slice blockIdx.y of a split-K launch (0 otherwise)
    GemmArgs a = a0;
    a.w += (size_t)blockIdx.y * a0.sw;
    a.x += (size_t)blockIdx.y * a0.sx;
    a.y += (size_t)blockIdx.y * a0.sy;
    constexpr int nt = NW * 64, nw = NW;
    const int tid = threadIdx.x, lane = tid & 63;
    const int w = tid >> 6;
    const int n_groups = a.out_dim / 32;
    int g = blockIdx.x;
    if (g >= n_groups) return;

    // the wave's X window as MFMA B operands (fp16), zero for vectors >= batch
    half8 xb[8 * NP];
    char* xs = lds + kRedOff + w * 16 * kRedRow * (int)sizeof(float);   // this wave's partial-tile area
    // Pipeline, one group ahead: group g's staged weights are taken into
    // registers, then the next group's staging loads go out and run during
    // g's products; g's pair table (slot j & 1) was built while group g-1
    // was multiplied, and the next group's table is built after the
    // products.  The LUT loads are issued before the weights, so the first
    // table build never waits for them.
    const int stride = gridDim.x;
    char* stage = lds + kRedOff + NW * 16 * kRedRow * (int)sizeof(float);
    float* red = reinterpret_cast<float*>(lds + kRedOff);
    uint32_t wa[12 * NP];
    if (g + stride >= n_groups) {
        // the only group of this workgroup: its stage overlays the partial
        // tiles, which are written only after the stage has been read; the
        // LUT loads go first so the table build does not wait for the weights
        char* stage1 = lds + kRedOff;
        stage_luts<nt>(a, lds, 0, tid);
        load_x<NP>(xb, a, xs, w, lane);
        lds_barrier();                                 // every wave is done with its x staging area
        stage_group<NW, NP>(a, g, stage1, w, lane);
        lds_barrier();
        build_table(lds, 0, 0, w, nw, lane);
        __builtin_amdgcn_s_waitcnt(0x0F70);            // this wave's staging loads landed
        lds_barrier();                                 // every wave's; table ready
        read_group<NW, NP>(wa, stage1, w, lane);
        lds_barrier();                                 // the stage is read: the partial tiles may overwrite it
        float16_t c = float16_t{};
        group_mfma<NP>(c, wa, xb, lds, 0u);
#pragma unroll
        for (int e = 0; e < 16; e++) red[w * 16 * kRedRow + red_pos(e, lane)] = c[e];
        lds_barrier();
        reduce_store<NW, ACC>(a, g, lds, tid);
        return;
    }
    stage_luts<nt>(a, lds, 0, tid);
    stage_group<NW, NP>(a, g, stage, w, lane);
    load_x<NP>(xb, a, xs, w, lane);
    lds_barrier();                                     // LUTs staged
    build_table(lds, 0, 0, w, nw, lane);
    for (int j = 0;; j++) {
        __builtin_amdgcn_s_waitcnt(0x0F70);            // this wave's staging loads of group g landed
        lds_barrier();                                 // every wave's; table j & 1 ready; red free
        read_group<NW, NP>(wa, stage, w, lane);
        lds_barrier();                                 // the stage is free
        const int gn = g + stride;
        if (gn < n_groups) stage_group<NW, NP>(a, gn, stage, w, lane);
        {
            float16_t c = float16_t{};
            group_mfma<NP>(c, wa, xb, lds, (uint32_t)((j & 1) * kTabBytes));
#pragma unroll
            for (int e = 0; e < 16; e++) red[w * 16 * kRedRow + red_pos(e, lane)] = c[e];
        }
        if (gn < n_groups) {
            if (((j + 1) & (kLutSlots - 1)) == 0) {
                // restage the next kLutSlots LUTs (every 64 groups of this workgroup)
                lds_barrier();
                stage_luts<nt>(a, lds, j + 1, tid);
                lds_barrier();
            }
            build_table(lds, (j + 1) & 1, j + 1, w, nw, lane);
        }
        lds_barrier();                                 // partial tiles complete
        reduce_store<NW, ACC>(a, g, lds, tid);
        g = gn;
        if (g >= n_groups) break;
    }
}

// y[i] = (y[i] if accumulate) + sum over the column slices of part[s][i].
__global__ __launch_bounds__(256) void split_sum_kernel(float* y, const float* part, long n, int nsplit, int accumulate) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = accumulate ? y[i] : 0.f;
    for (int k = 0; k < nsplit; k++) s += part[(long)k * n + i];
    y[i] = s;
}

// split_sum_kernel for one row per workgroup (rows of out_dim <= 4 * 1024
// elements, up to 16 column slices), followed by the RMSNorm of the summed row
// times w into xn (cpu_ops.cpp:24-30): the norm input of the next layer's
// FFN, one launch fewer.  Each thread issues all of its loads at once (the
// slices unrolled), then adds them in slice order.
constexpr int kSumNormThreads = 1024, kSumNormReg = 4, kSumNormSplits = 16;
__global__ __launch_bounds__(kSumNormThreads) void split_sum_norm_kernel(float* y, const float* part, float* xn,
                                                                         const float* w, int out_dim, long n,
                                                                         int nsplit, int accumulate, float eps) {
    constexpr int NT = kSumNormThreads, R = kSumNormReg, S = kSumNormSplits;
    __shared__ float red[NT / 64];
    const size_t r0 = (size_t)blockIdx.x * out_dim;
    float v[R], wv[R];
#pragma unroll
    for (int k = 0; k < R; k++) {
        const int i = threadIdx.x + NT * k;
        const bool in = i < out_dim;
        const size_t e = r0 + (in ? i : 0);
        float ps[S];
#pragma unroll
        for (int sp = 0; sp < S; sp++) ps[sp] = sp < nsplit ? part[(long)sp * n + e] : 0.f;
        float s = accumulate ? y[e] : 0.f;
#pragma unroll
        for (int sp = 0; sp < S; sp++)
            if (sp < nsplit) s += ps[sp];
        if (in) y[e] = s;
        v[k] = in ? s : 0.f;
        wv[k] = in ? w[i] : 0.f;
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < R; k++) ss += v[k] * v[k];
    ss = block_sum<NT>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)out_dim + eps);
#pragma unroll
    for (int k = 0; k < R; k++) {
        const int i = threadIdx.x + NT * k;
        if (i < out_dim) xn[r0 + i] = (v[k] * inv) * wv[k];
    }
}

}  // namespace

bool lut6_split_sum_norm_fits(int out_dim, int nsplit) {
    return out_dim <= kSumNormThreads * kSumNormReg && nsplit <= kSumNormSplits;
}
int lut6_split_sum_norm(float* y, const float* part, long n, int nsplit, int accumulate, int rows, int out_dim,
                        const float* norm_w, float eps, float* xn, hipStream_t st) {
    if (out_dim > kSumNormThreads * kSumNormReg || nsplit > kSumNormSplits)
        return set_error(ANELM_EINVAL, "split_sum_norm: row of %d elements in %d slices", out_dim, nsplit);
    hipLaunchKernelGGL(split_sum_norm_kernel, dim3((unsigned)rows), dim3(kSumNormThreads), 0, st, y, part, xn, norm_w,
                       out_dim, n, nsplit, accumulate, eps);
    ANELM_LAUNCHED("split_sum_norm_kernel");
    return ANELM_OK;
}

int lut6_split_sum(float* y, const float* part, long n, int nsplit, int accumulate, hipStream_t st) {
    hipLaunchKernelGGL(split_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, part, n, nsplit,
                       accumulate);
    ANELM_LAUNCHED("split_sum_kernel");
    return ANELM_OK;
}

// Column split for the GEMM: NP (1 or 2) and the wave count in_dim / (128 NP).
// NP = 2 (256 columns per wave) up to 10 waves; otherwise NP = 1 (128 columns
// per wave, an odd number of waves up to 15).
bool lut6_gemm_geometry(int in_dim, int& np, int& waves) {
    if (in_dim % 256 == 0 && in_dim / 256 <= 10) {
        np = 2;
        waves = in_dim / 256;
        return true;
    }
    if (in_dim % 128 == 0 && (in_dim / 128) % 2 == 1 && in_dim / 128 <= 15) {
        np = 1;
        waves = in_dim / 128;
        return true;
    }
    return false;
}

// Y[b][r] for b < batch (batch <= 32), out_dim % 32 == 0, in_dim accepted by
// lut6_gemm_geometry.  Shapes are validated by the caller.
int lut6_gemm_launch(float* y, const uint8_t* w, long ldw, const uint16_t* lut, const float* x, long ldx, int batch,
                     int out_dim, int in_dim, int accumulate, int nsplit, long sy, hipStream_t st) {
    int np = 0, waves = 0;
    if (!lut6_gemm_geometry(in_dim, np, waves) || batch < 1 || batch > 32 || out_dim % 32 ||
        (long long)batch * out_dim * 4 >= (1LL << 31) || (long long)(out_dim + 32 * 1024) * ldw >= (1LL << 31))
        return set_error(ANELM_EINVAL, "lut6_gemm: unsupported shape batch %d out %d in %d", batch, out_dim,
                         in_dim);
    Device* dev = device();
    if (!dev) return ANELM_EHIP;
    GemmArgs a{y, w, lut, x, batch, out_dim, in_dim, ldw, ldx, accumulate,
               (long)in_dim * 3 / 4, (long)in_dim, sy};
    const int n_groups = out_dim / 32;
    // a grid-stride walk over the groups with about one workgroup per CU in
    // all: each workgroup loads its window of the inputs once for all its
    // groups (a split launch has nsplit column slices of the grid)
    int grid = n_groups;
    const int per_slice = std::max(1, dev->num_cus / nsplit);
    if (grid > per_slice) grid = per_slice;
    // a workgroup with one group overlays its stage on the partial tiles
    const size_t red_bytes = (size_t)waves * 16 * kRedRow * sizeof(float);
    const size_t stage_bytes = np == 2 ? (32 * (waves * 192 / 16 + 1) + 63) / 64 * 1024
                                       : (32 * (waves * 96 / 16 + 1) + 63) / 64 * 1024;
    const size_t lds = (size_t)kRedOff + (grid == n_groups ? std::max(red_bytes, stage_bytes) : red_bytes + stage_bytes);
    using K = void (*)(GemmArgs);
#define ANELM_K2(A) {nullptr, lut6_gemm_kernel<2, 1, A>, lut6_gemm_kernel<2, 2, A>, lut6_gemm_kernel<2, 3, A>,     \
                     lut6_gemm_kernel<2, 4, A>, lut6_gemm_kernel<2, 5, A>, lut6_gemm_kernel<2, 6, A>,              \
                     lut6_gemm_kernel<2, 7, A>, lut6_gemm_kernel<2, 8, A>, lut6_gemm_kernel<2, 9, A>,              \
                     lut6_gemm_kernel<2, 10, A>}
#define ANELM_K1(A) {nullptr, lut6_gemm_kernel<1, 1, A>, nullptr, lut6_gemm_kernel<1, 3, A>, nullptr,              \
                     lut6_gemm_kernel<1, 5, A>, nullptr, lut6_gemm_kernel<1, 7, A>, nullptr,                         \
                     lut6_gemm_kernel<1, 9, A>, nullptr, lut6_gemm_kernel<1, 11, A>, nullptr,                        \
                     lut6_gemm_kernel<1, 13, A>, nullptr, lut6_gemm_kernel<1, 15, A>}
    static const K k2[2][11] = {ANELM_K2(false), ANELM_K2(true)};
    static const K k1[2][16] = {ANELM_K1(false), ANELM_K1(true)};
#undef ANELM_K2
#undef ANELM_K1
    const int acc = accumulate ? 1 : 0;
    const K kp = np == 2 ? k2[acc][waves] : k1[acc][waves];
    if (!kp) return set_error(ANELM_EINVAL, "lut6_gemm: no kernel for %d waves (np %d)", waves, np);
    // the attribute covers the staged size (the larger of the two per kernel)
    static bool attr_set[2][2][16] = {};
    if (!attr_set[acc][np - 1][waves]) {
        const int full = (int)((size_t)kRedOff + red_bytes + stage_bytes);
        ANELM_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kp), hipFuncAttributeMaxDynamicSharedMemorySize,
                                      full));
        attr_set[acc][np - 1][waves] = true;
    }
    hipLaunchKernelGGL(kp, dim3(grid, nsplit), dim3(waves * 64), lds, st, a);
    ANELM_LAUNCHED("lut6_gemm_kernel");
    return ANELM_OK;
}

}  // namespace anelm
