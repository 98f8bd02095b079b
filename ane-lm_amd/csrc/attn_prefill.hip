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
// permuted identically in both operands).  K and V tiles of 32 keys are
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

// Query row r is key qoff + r of the L keys in k / v (the keys before qoff
// are a cached prefix) and attends keys (qoff + r - win, qoff + r] (win 0: no
// lower bound).  With gate, the output row is multiplied by sigmoid of
// gate[r * gtok + h * ghead + d] (the reference's output gate).
template <int D, int HB, int RB, bool OUT16>
__global__ __launch_bounds__(HB * RB * 64) void prefill_kernel(void* out, const _Float16* q,
                                                               const _Float16* k, const _Float16* v,
                                                               int S, int L, int qoff, int win, int Hq, int Hkv,
                                                               const float* gate, int gtok, int ghead) {
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

    const int nkt = (qoff + row_end + kBN - 1) / kBN;
    // first tile any row of the workgroup sees
    const int kt0 = win > 0 ? max(0, qoff + qt * RB * 32 + 1 - win) / kBN : 0;
    for (int kt = kt0; kt < nkt; kt++) {
        const int j0 = kt * kBN;
        __syncthreads();
        for (int c = tid; c < kBN * D / 8; c += NT) {
            const int kr = c / (D / 8), kc = (c % (D / 8)) * 8;
            const int key = j0 + kr;
            uint4 kv4 = make_uint4(0, 0, 0, 0), vv4 = make_uint4(0, 0, 0, 0);
            if (key < L) {
                kv4 = *reinterpret_cast<const uint4*>(k + ((size_t)key * Hkv + kvh) * D + kc);
                vv4 = *reinterpret_cast<const uint4*>(v + ((size_t)key * Hkv + kvh) * D + kc);
            }
            *reinterpret_cast<uint4*>(&Ks[kr][kc]) = kv4;
            const _Float16* vh = reinterpret_cast<const _Float16*>(&vv4);
#pragma unroll
            for (int i = 0; i < 8; i++) Vt[kc + i][kr] = vh[i];
        }
        __syncthreads();
        // wave-uniform: every key of the tile after the wave's rows, or (with
        // a window) before the window of its first row
        if (q0 >= S || j0 > qoff + q0 + 31 || (win > 0 && j0 + kBN <= qoff + q0 + 1 - win)) continue;

        float16_t s = float16_t{};
#pragma unroll
        for (int ks = 0; ks < KS; ks++) {
            const half8 a = *reinterpret_cast<const half8*>(&Ks[r][16 * ks + 8 * hh]);
            s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qf[ks], s, 0, 0, 0);
        }
        // s[e] = score of key j0 + 8*(e/4) + 4*hh + e%4 for query row qrow
        float mx = -INFINITY;
        const int kmax = qoff + qrow, kmin = win > 0 ? qoff + qrow - win : -1;
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int key = j0 + 8 * (e / 4) + 4 * hh + (e % 4);
            const float val = (key <= kmax && key > kmin) ? s[e] * sl2 : -INFINITY;
            s[e] = val;
            mx = fmaxf(mx, val);
        }
        mx = fmaxf(mx, shfl_xor(mx, 32));
        // a row that has seen no key yet (below its window) keeps m = -inf:
        // its terms are exp2(-inf) = 0 against a finite reference
        const float m_new = fmaxf(m, mx);
        const float m_ref = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp2f(m - m_ref);
        float ps = 0.f;
        half8 pf[2];
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const float pe = exp2f(s[e] - m_ref);
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
            float a0 = o[db][4 * g4] * inv, a1 = o[db][4 * g4 + 1] * inv;
            float a2 = o[db][4 * g4 + 2] * inv, a3 = o[db][4 * g4 + 3] * inv;
            if (gate) {
                const float* gr = gate + (size_t)qrow * gtok + (size_t)h * ghead + d;
                a0 = a0 / (1.0f + expf(-gr[0]));
                a1 = a1 / (1.0f + expf(-gr[1]));
                a2 = a2 / (1.0f + expf(-gr[2]));
                a3 = a3 / (1.0f + expf(-gr[3]));
            }
            if (OUT16) {
                half4 hv = {(_Float16)a0, (_Float16)a1, (_Float16)a2, (_Float16)a3};
                *reinterpret_cast<half4*>(static_cast<_Float16*>(out) + off) = hv;
            } else {
                *reinterpret_cast<float4*>(static_cast<float*>(out) + off) = make_float4(a0, a1, a2, a3);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Workload-balanced, pipelined kernel for head_dim 256 and 4 query heads per KV
// head (the Qwen3.5 shapes).
//
// * Blocks of 64 query rows; a workgroup's 8 waves are 4 query heads x 2 row
//   halves of 32 rows, and all of them consume ONE stream of 32-key tiles, so
//   each K / V byte staged in LDS feeds 256 query rows.
// * Balance: a unit is a KV head and a pair of blocks (a, nb-1-a) (or the
//   middle block when nb is odd).  Its causal key tiles, a's then b's, are cut
//   into two equal halves taken by two workgroups.  The block whose tiles are
//   split is merged by whichever of the two finishes second: a relaxed
//   device-scope counter orders their arrivals, the first writes its partial
//   (m, l, unnormalised O) with device-coherent stores and counts again once
//   they are out, the second waits for that count, combines the partial with
//   its registers, writes the rows and re-zeroes the counter for the next
//   call.
// * Stream: K and V tiles (32 keys x 256) go straight to LDS with buffer loads
//   (1 KiB per wave instruction: rows c and c+16 of a tile share a chunk) into
//   a ring of 4 buffers, 3 tiles ahead of use.  K chunks are 1040 bytes (16 of
//   padding) so the MFMA operand reads are conflict-free with immediate
//   offsets; V chunks are 1088 bytes, so the four key rows a 16-lane group
//   reads with ds_read_b64_tr_b16 (4 keys x 16 dims, delivered transposed:
//   lane n gets dim n of the 4 keys) fall on distinct banks.  That transposing
//   read builds the V^T operand of O^T += V^T P^T from the V rows as stored.
// * Scores S^T = K Q^T (v_mfma_f32_32x32x16_f16).  The A-operand lane i reads
//   key row pi(i) (bits 2 and 3 of i swapped): lane (r, h) of the accumulator
//   then holds the scores of query row r for keys 8h..8h+7 and 16+8h..16+8h+7,
//   exactly the B-operand keys of O^T += V^T P^T.
// * Softmax in the log2 domain; the running maximum only moves when it grows
//   by more than 8, so probabilities stay below 2^8 (fp16-exact range) and the
//   128-register output rescale is rare.
constexpr int kGKeys = 32;                       // keys per tile
constexpr int kGKBytes = 16 * 1040;              // K tile: chunk c = rows c, c + 16
constexpr int kGVChunk = 1088;                   // V tile chunk: rows c, c + 16 + 64 bytes of bank offset
constexpr int kGTile = kGKBytes + 16 * kGVChunk; // + V tile (32 x 256 fp16)
constexpr int kGBuf = 4;                         // ring of tile buffers
constexpr int kGLds = kGBuf * kGTile + 64;       // + the merge flag
constexpr int kGSlotFloats = 8 * 128 * 64 + 8 * 128;   // partial: O (8 waves x 128 x 64 lanes), m, l
constexpr int kGNT = 512;
constexpr int kSc1 = 16;                         // buffer cache policy: device-scope coherent

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ int key_perm(int i) { return (i & ~12) | ((i & 4) << 1) | ((i & 8) >> 1); }

// Key tiles needed by 64-row block blk: keys 0 .. qoff + min(64 blk + 63, S - 1).
__device__ __forceinline__ int block_tiles(int blk, int S, int qoff) {
    return (qoff + min(64 * blk + 64, S) + 31) / 32;
}

// Query row r is key qoff + r of the L keys (the keys before qoff are a
// cached prefix) and attends keys 0 .. qoff + r.  With gate, output row
// (r, h) is multiplied by sigmoid(gate[r * gtok + h * ghead + d]).
template <bool OUT16, bool GATE>
__global__ __launch_bounds__(kGNT) void prefill_g4_kernel(void* out, const _Float16* q, const _Float16* k,
                                                           const _Float16* v, float* part, uint32_t* ctr, int S,
                                                           int L, int qoff, int Hq, int Hkv,
                                                           const float* gate, int gtok, int ghead) {
    constexpr int D = 256, KS = D / 16, DB = D / 32;
    extern __shared__ __attribute__((aligned(16))) char lds[];
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hl = w & 3, rh = w >> 2;
    const int nb = (S + 63) / 64, npair = nb / 2, upk = npair + (nb & 1);
    // consecutive units on one XCD (workgroup id mod 8 selects the XCD): one KV head per L2
    int lw = blockIdx.x;
    if (gridDim.x % 8 == 0) lw = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
    const int unit = lw >> 1, half_id = lw & 1;
    const int kvh = unit / upk, pu = unit % upk;
    const int h = kvh * 4 + hl;
    const int blk_a = pu < npair ? pu : -1, blk_b = pu < npair ? nb - 1 - pu : npair;
    const int nta = blk_a >= 0 ? block_tiles(blk_a, S, qoff) : 0, ntb = block_tiles(blk_b, S, qoff);
    const int half = (nta + ntb) / 2, nb0 = half - nta;   // tiles of b taken by the first workgroup
    const bool split = nb0 > 0;
    // this workgroup's segments (block, first key tile, tile count)
    int blk0, t00, n0, blk1 = 0, t01 = 0, n1 = 0;
    if (half_id == 0) {
        if (nta > 0) {
            blk0 = blk_a; t00 = 0; n0 = nta;
            if (nb0 > 0) { blk1 = blk_b; t01 = 0; n1 = nb0; }
        } else {
            blk0 = blk_b; t00 = 0; n0 = nb0;
        }
    } else {
        const int f = nb0 > 0 ? nb0 : 0;
        blk0 = blk_b; t00 = f; n0 = ntb - f;
    }
    if (n0 <= 0) return;
    const int nseg = n1 > 0 ? 2 : 1;
    const int ntot = n0 + n1;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(k), 0, (int)min((size_t)L * Hkv * D * 2, (size_t)0x7fffffff), 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<_Float16*>(v), 0, (int)min((size_t)L * Hkv * D * 2, (size_t)0x7fffffff), 0x00020000);
    const float sl2 = (1.0f / 16.0f) * 1.4426950408889634f;   // 1/sqrt(256) * log2(e)
    auto key_tile = [&](int i) { return i < n0 ? t00 + i : t01 + (i - n0); };
    // stream tile i -> buffer i % 4; wave w loads K and V chunks 2w, 2w+1
    auto issue = [&](int i) {
        char* base = lds + (i % kGBuf) * kGTile;
        const int j0 = key_tile(i) * kGKeys;
        int ln = threadIdx.x & 63;
        asm volatile("" : "+v"(ln));   // lane offsets are recomputed here, not held across the loop
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int c = 2 * w + x, row = c + 16 * (ln >> 5), key = j0 + row;
            const int off = key < L ? ((key * Hkv + kvh) * D + 8 * (ln & 31)) * 2 : 0x7fffffff;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (__attribute__((address_space(3))) void*)(base + c * 1040), 16,
                                                     off, 0, 0, 0);
        }
#pragma unroll
        for (int x = 0; x < 2; x++) {
            const int c = 2 * w + x, row = c + 16 * (ln >> 5), key = j0 + row;
            const int off = key < L ? ((key * Hkv + kvh) * D + 8 * (ln & 31)) * 2 : 0x7fffffff;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rv, (__attribute__((address_space(3))) void*)(base + kGKBytes + c * kGVChunk), 16, off, 0, 0, 0);
        }
    };
    for (int i = 0; i < 3 && i < ntot; i++) issue(i);
    int i = 0;
    for (int sg = 0; sg < nseg; sg++) {
        const int blk = sg == 0 ? blk0 : blk1;
        const int row0 = 64 * blk + 32 * rh;
        half8 qf[KS];
        {
            const int lane = threadIdx.x & 63, qrow = row0 + (lane & 31);
#pragma unroll
            for (int ks = 0; ks < KS; ks++) {
                if (qrow < S)
                    qf[ks] = *reinterpret_cast<const half8*>(q + ((size_t)qrow * Hq + h) * D + 16 * ks + 8 * (lane >> 5));
                else
                    qf[ks] = half8{};
            }
        }
        // the Q fragments complete here, so no wait for them remains inside the tile loop
        __builtin_amdgcn_s_waitcnt(0x0F70);
        float16_t o[DB];
#pragma unroll
        for (int db = 0; db < DB; db++) o[db] = float16_t{};
        float m = -INFINITY, l = 0.f;
        const int iend = sg == 0 ? n0 : ntot;
        for (; i < iend; i++) {
            // tile i has landed once at most the loads of tiles i+1, i+2 (4 per wave each) remain
            const int left = ntot - 1 - i;
            if (left >= 2) __builtin_amdgcn_s_waitcnt(0x0F78);
            else if (left == 1) __builtin_amdgcn_s_waitcnt(0x0F74);
            else __builtin_amdgcn_s_waitcnt(0x0F70);
            __syncthreads();   // every wave's part of tile i landed; buffer (i+3)%4 (tile i-1) is free
            if (i + 3 < ntot) issue(i + 3);
            const int kt = key_tile(i), j0 = kt * kGKeys;
            if (j0 > qoff + row0 + 31) continue;   // every key of this tile lies after this wave's rows
            const char* base = lds + (i % kGBuf) * kGTile;
            int ln = threadIdx.x & 63;
            asm volatile("" : "+v"(ln));
            // ---- S^T = K Q^T
            float16_t sc = float16_t{};
            {
                const int krow = key_perm(ln & 31);
                const char* kb = base + (krow & 15) * 1040 + (krow >> 4) * 512 + (ln >> 5) * 16;
#pragma unroll
                for (int ks = 0; ks < KS; ks++)
                    sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(*reinterpret_cast<const half8*>(kb + 32 * ks), qf[ks], sc,
                                                                0, 0, 0);
                // K fragment ks + 1 is read while the product of fragment ks runs
                __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
                for (int ks = 0; ks < KS - 2; ks++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
            }
            // ---- online softmax; element e holds key j0 + (e < 8 ? 8 h + e : 16 + 8 h + e - 8)
            if (j0 + 31 > qoff + row0) {
                const int h2 = ln >> 5, qr = qoff + row0 + (ln & 31);
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int key = j0 + (e < 8 ? 8 * h2 + e : 16 + 8 * h2 + (e - 8));
                    sc[e] = key <= qr ? sc[e] : -INFINITY;
                }
            }
            float mx = -INFINITY;
#pragma unroll
            for (int e = 0; e < 16; e++) mx = fmaxf(mx, sc[e]);
            mx = fmaxf(mx, shfl_xor(mx, 32)) * sl2;
            if (__builtin_amdgcn_ballot_w64(mx > m + 8.0f) != 0) {
                const float m_new = fmaxf(m, mx);
                const float alpha = __builtin_amdgcn_exp2f(m - m_new);
                l *= alpha;
#pragma unroll
                for (int db = 0; db < DB; db++)
#pragma unroll
                    for (int e = 0; e < 16; e++) o[db][e] *= alpha;
                m = m_new;
            }
            half8 pf[2];
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float pe = __builtin_amdgcn_exp2f(fmaf(sc[e], sl2, -m));
                l += pe;
                pf[e / 8][e % 8] = (_Float16)pe;
            }
            // ---- O^T += V^T P^T.  The A operand of lane (m, h2) for keys
            // 16u + 8 h2 .. +8 and dim 32 db + m comes from two transposing
            // reads: 16-lane group i (m = 16 (i & 1) + n, h2 = i >> 1) has
            // its lane n address key 16u + 8 (i >> 1) + 4r + n / 4, dims
            // 32 db + 16 (i & 1) + 4 (n % 4) .. +4 of the V rows (key t at
            // chunk t % 16, half t / 16).
            {
                const int gi = ln >> 4, nn = ln & 15;
                const char* vbase = base + kGKBytes + (8 * (gi >> 1) + (nn >> 2)) * kGVChunk +
                                    (16 * (gi & 1) + 4 * (nn & 3)) * 2;
                typedef short s16x4 __attribute__((ext_vector_type(4)));
                static_assert(4 * kGVChunk == 4352, "offset of the second read");
                const uint32_t va = (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const char*)vbase);
                // product k = 2 db + u; the reads of product k + 1 are issued
                // before product k (each asm statement waits only for the
                // older pair, which it passes through to the product)
                s16x4 lo[2], hi[2];
                asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %2 offset:4352"
                             : "=&v"(lo[0]), "=&v"(hi[0])
                             : "v"(va)
                             : "memory");
#pragma unroll
                for (int kk = 0; kk < 2 * DB; kk++) {
                    const int db = kk >> 1, u = kk & 1, c = kk & 1, n = c ^ 1;
                    if (kk + 1 < 2 * DB) {
                        const int u1 = (kk + 1) & 1, db1 = (kk + 1) >> 1;
                        asm volatile(
                            "ds_read_b64_tr_b16 %0, %4\n\tds_read_b64_tr_b16 %1, %4 offset:4352\n\ts_waitcnt lgkmcnt(2)"
                            : "=&v"(lo[n]), "=&v"(hi[n]), "+v"(lo[c]), "+v"(hi[c])
                            : "v"(va + (uint32_t)(u1 * 512 + 64 * db1))
                            : "memory");
                    } else {
                        asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(lo[c]), "+v"(hi[c]) : : "memory");
                    }
                    const half8 av =
                        __builtin_bit_cast(half8, __builtin_shufflevector(lo[c], hi[c], 0, 1, 2, 3, 4, 5, 6, 7));
                    o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, pf[u], o[db], 0, 0, 0);
                }
            }
        }
        l += shfl_xor(l, 32);
        int ln = threadIdx.x & 63;
        asm volatile("" : "+v"(ln));   // the epilogue's addresses are computed here, not held through the loop
        const int erow = row0 + (ln & 31), eh = ln >> 5;
        float a0 = 1.f, a1 = 0.f, inv;
        __amdgpu_buffer_rsrc_t rot = __builtin_amdgcn_make_buffer_rsrc(part, 0, 0, 0x00020000);
        bool have_other = false;
        if (split && blk == blk_b) {
            // The split block's two workgroups arrive on the unit's counter
            // (0 -> 1 -> 2, one more when the first one's partial is out).
            // The first to arrive publishes its partial and leaves; the
            // second waits until that partial is stored (the first is
            // resident, and nothing stands between its arrival and its
            // stores), merges it with its own registers and re-zeroes the
            // counter.  One partial per split block is written and read.
            uint32_t* flag = reinterpret_cast<uint32_t*>(lds + kGBuf * kGTile);
            if (tid == 0) flag[0] = __hip_atomic_fetch_add(&ctr[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            const uint32_t arrived = flag[0];
            rot = __builtin_amdgcn_make_buffer_rsrc(part + (size_t)unit * kGSlotFloats, 0, kGSlotFloats * 4, 0x00020000);
            if (arrived == 0) {
#pragma unroll
                for (int db = 0; db < DB; db++)
#pragma unroll
                    for (int g4 = 0; g4 < 4; g4++) {
                        const float4 v4 =
                            make_float4(o[db][4 * g4], o[db][4 * g4 + 1], o[db][4 * g4 + 2], o[db][4 * g4 + 3]);
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v4), rot,
                                                               (((w * DB + db) * 4 + g4) * 256 + ln * 4) * 4, 0, kSc1);
                    }
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, m), rot,
                                                      (8 * 128 * 64 + w * 128 + ln) * 4, 0, kSc1);
                __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, l), rot,
                                                      (8 * 128 * 64 + w * 128 + 64 + ln) * 4, 0, kSc1);
                __builtin_amdgcn_s_waitcnt(0x0F70);   // this wave's part of the partial is stored
                __syncthreads();
                if (tid == 0) __hip_atomic_fetch_add(&ctr[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;   // the other workgroup finishes this block (its segment is the last)
            }
            if (tid == 0) {
                // bounded: the first workgroup only has its stores left
                uint32_t c = arrived + 1;
                for (int it = 0; c != 3 && it < (1 << 22); it++) {
                    __builtin_amdgcn_s_sleep(2);
                    c = __hip_atomic_load(&ctr[unit], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __hip_atomic_store(&ctr[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            have_other = true;
            const float m1 = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rot, (8 * 128 * 64 + w * 128 + ln) * 4, 0, kSc1));
            const float l1 = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rot, (8 * 128 * 64 + w * 128 + 64 + ln) * 4, 0, kSc1));
            const float M = fmaxf(m, m1);
            a0 = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
            a1 = m1 == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m1 - M);
            {
#pragma clang fp contract(off)
                inv = 1.0f / (l * a0 + l1 * a1);
            }
        } else {
            inv = 1.0f / l;
        }
        if (erow < S) {
            // o[db][e] = output dim 32 db + 8 (e / 4) + 4 h + e % 4 of row erow.
            // The other partial's values and the gate logits of column block
            // db + 1 are requested before the stores of block db: issued after
            // them, each request would wait for those stores (the output may
            // alias them as far as the compiler knows).
            const float* grow = GATE ? gate + (size_t)erow * gtok + (size_t)h * ghead : nullptr;
            auto fetch = [&](int db, float4 (&ov)[4], float4 (&gv)[4]) __attribute__((always_inline)) {
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int dd = 32 * db + 8 * g4 + 4 * eh;
                    ov[g4] = make_float4(0.f, 0.f, 0.f, 0.f);
                    gv[g4] = make_float4(0.f, 0.f, 0.f, 0.f);
                    if (have_other)
                        ov[g4] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                rot, (((w * DB + db) * 4 + g4) * 256 + ln * 4) * 4, 0, kSc1));
                    if constexpr (GATE)   // (rows of any stride: four dword loads)
                        gv[g4] = make_float4(grow[dd], grow[dd + 1], grow[dd + 2], grow[dd + 3]);
                }
            };
            float4 ovn[4], gvn[4];
            fetch(0, ovn, gvn);
#pragma unroll
            for (int db = 0; db < DB; db++) {
                float4 ovc[4], gvc[4];
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    ovc[g4] = ovn[g4];
                    gvc[g4] = gvn[g4];
                }
                if (db + 1 < DB) fetch(db + 1, ovn, gvn);
#pragma unroll
                for (int g4 = 0; g4 < 4; g4++) {
                    const int dd = 32 * db + 8 * g4 + 4 * eh;
                    const size_t off = ((size_t)erow * Hq + h) * D + dd;
                    const float4 ov = ovc[g4];
                    float v0, v1, v2, v3;
                    {
                        // Either workgroup of a split block may be the one that
                        // merges: products rounded separately keep the sum
                        // symmetric in the two partials, so a row's bits do not
                        // depend on which finished second.
#pragma clang fp contract(off)
                        v0 = (o[db][4 * g4] * a0 + ov.x * a1) * inv;
                        v1 = (o[db][4 * g4 + 1] * a0 + ov.y * a1) * inv;
                        v2 = (o[db][4 * g4 + 2] * a0 + ov.z * a1) * inv;
                        v3 = (o[db][4 * g4 + 3] * a0 + ov.w * a1) * inv;
                    }
                    if constexpr (GATE) {
                        const float4 gl = gvc[g4];
                        v0 = v0 / (1.0f + expf(-gl.x));
                        v1 = v1 / (1.0f + expf(-gl.y));
                        v2 = v2 / (1.0f + expf(-gl.z));
                        v3 = v3 / (1.0f + expf(-gl.w));
                    }
                    if (OUT16) {
                        half4 hv = {(_Float16)v0, (_Float16)v1, (_Float16)v2, (_Float16)v3};
                        *reinterpret_cast<half4*>(static_cast<_Float16*>(out) + off) = hv;
                    } else {
                        *reinterpret_cast<float4*>(static_cast<float*>(out) + off) = make_float4(v0, v1, v2, v3);
                    }
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0x0F70);   // stores retired before the stream's counted waits resume
    }
}

int launch_prefill_g4(void* out, bool out16, const void* q, const void* k, const void* v, int S, int L, int qoff,
                      int Hq, int Hkv, const float* gate, int gtok, int ghead, hipStream_t st) {
    constexpr int D = 256;
    ANELM_REQUIRE((size_t)L * Hkv * D * 2 < 0x7fffffffu, "prefill: %d keys exceed the 2 GiB buffer range", L);
    const int nb = (S + 63) / 64, upk = nb / 2 + (nb & 1), units = Hkv * upk;
    const size_t part_bytes = (size_t)units * kGSlotFloats * sizeof(float);
    float* part = static_cast<float*>(workspace(part_bytes, st));
    if (!part) return ANELM_ENOMEM;
    uint32_t* ctr = counters(units, kCtrPrefill, st);   // zeroed; each call leaves them zeroed
    if (!ctr) return ANELM_ERANGE;
    // the gated launches (prompt prefill through the layer core) are their own
    // instantiation: the bare core carries no gate code
    using K = void (*)(void*, const _Float16*, const _Float16*, const _Float16*, float*, uint32_t*, int, int, int,
                       int, int, const float*, int, int);
    static const K kern[2][2] = {{prefill_g4_kernel<false, false>, prefill_g4_kernel<false, true>},
                                 {prefill_g4_kernel<true, false>, prefill_g4_kernel<true, true>}};
    static bool attr_set = false;
    if (!attr_set) {
        for (int o = 0; o < 2; o++)
            for (int g = 0; g < 2; g++)
                ANELM_HIP(hipFuncSetAttribute(reinterpret_cast<const void*>(kern[o][g]),
                                              hipFuncAttributeMaxDynamicSharedMemorySize, kGLds));
        attr_set = true;
    }
    const _Float16* qh = static_cast<const _Float16*>(q);
    const _Float16* kh = static_cast<const _Float16*>(k);
    const _Float16* vh = static_cast<const _Float16*>(v);
    const dim3 grid(2 * units);
    hipLaunchKernelGGL(kern[out16 ? 1 : 0][gate != nullptr ? 1 : 0], grid, dim3(kGNT), kGLds, st, out, qh, kh, vh,
                       part, ctr, S, L, qoff, Hq, Hkv, gate, gtok, ghead);
    ANELM_LAUNCHED("prefill_g4_kernel");
    return ANELM_OK;
}

template <int D, int HB, int RB>
int launch_prefill(void* out, bool out16, const void* q, const void* k, const void* v, int S, int L, int qoff,
                   int win, int Hq, int Hkv, const float* gate, int gtok, int ghead, hipStream_t st) {
    const int rows = 32 * RB;
    dim3 grid((S + rows - 1) / rows, Hq / HB), block(HB * RB * 64);
    const _Float16* qh = static_cast<const _Float16*>(q);
    const _Float16* kh = static_cast<const _Float16*>(k);
    const _Float16* vh = static_cast<const _Float16*>(v);
    if (out16)
        hipLaunchKernelGGL((prefill_kernel<D, HB, RB, true>), grid, block, 0, st, out, qh, kh, vh, S, L, qoff, win,
                           Hq, Hkv, gate, gtok, ghead);
    else
        hipLaunchKernelGGL((prefill_kernel<D, HB, RB, false>), grid, block, 0, st, out, qh, kh, vh, S, L, qoff, win,
                           Hq, Hkv, gate, gtok, ghead);
    ANELM_LAUNCHED("prefill_kernel");
    return ANELM_OK;
}

template <int D>
int dispatch_g(void* out, bool out16, const void* q, const void* k, const void* v, int S, int L, int qoff, int win,
               int Hq, int Hkv, const float* gate, int gtok, int ghead, hipStream_t st) {
    switch (Hq / Hkv) {
        case 1: return launch_prefill<D, 1, 8>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        case 2: return launch_prefill<D, 2, 4>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        case 4:
            // the pipelined kernel walks every key from 0: no window
            if (D == 256 && win == 0)
                return launch_prefill_g4(out, out16, q, k, v, S, L, qoff, Hq, Hkv, gate, gtok, ghead, st);
            return launch_prefill<D, 4, 2>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        case 8: return launch_prefill<D, 4, 2>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        default: return set_error(ANELM_EINVAL, "prefill: n_heads/n_kv_heads = %d unsupported", Hq / Hkv);
    }
}

}  // namespace

int prefill_core(void* out, bool out16, const uint16_t* q, const uint16_t* k, const uint16_t* v, int S, int L,
                 int qoff, int win, int Hq, int Hkv, int D, const float* gate, int gtok, int ghead, hipStream_t st) {
    switch (D) {
        case 128: return dispatch_g<128>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        case 256: return dispatch_g<256>(out, out16, q, k, v, S, L, qoff, win, Hq, Hkv, gate, gtok, ghead, st);
        default: return set_error(ANELM_EINVAL, "prefill: head_dim %d unsupported (128, 256)", D);
    }
}

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
    return prefill_core(out, out_dtype == ANELM_F16, q, k, v, S, S, 0, 0, n_heads, n_kv_heads, head_dim, nullptr, 0,
                        0, as_stream(stream));
}
