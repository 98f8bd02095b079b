// anelm_full_attn_decode_noalloc: the fused full-attention decode step of
// attn_decode.hip with its split partials in a file-scope device array, so a
// call allocates nothing (no hipMalloc / hipFree, no library workspace, no
// per-device library state).
#include "anelm_internal.hpp"

#include <mutex>

namespace anelm {

// ------------------------------------------------------ allocation-free entry
// Split partials of anelm_full_attn_decode_noalloc live in this file-scope
// device array (each device holds its own copy for the life of the process);
// its last 1 KiB holds the arrival counters of the in-kernel split merge,
// zero at load and left zero by every call.
// Host code never uses the symbol itself as an address: the array's device
// address is looked up once per device with hipGetSymbolAddress and kept in
// g_scratch_ptr.  Calls that overlap on one device share the array and race.
constexpr size_t kScratchBytes = (size_t)8 << 20;
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

static constexpr int kScratchDevices = 64;
static float* g_scratch_ptr[kScratchDevices];
static std::mutex g_scratch_mu;

// Device address of this device's scratch array; nullptr with the error
// recorded on failure.  Allocates nothing.
static float* scratch_ptr() {
    int id = 0;
    hipError_t e = hipGetDevice(&id);
    if (e != hipSuccess) { hip_fail(e, "hipGetDevice"); return nullptr; }
    if (id < 0 || id >= kScratchDevices) { set_error(ANELM_ERANGE, "device %d out of range", id); return nullptr; }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (g_scratch_ptr[id] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) { hip_fail(e, "hipGetSymbolAddress(scratch)"); return nullptr; }
        g_scratch_ptr[id] = static_cast<float*>(p);
    }
    return g_scratch_ptr[id];
}

}  // namespace anelm

using namespace anelm;

extern "C" int anelm_full_attn_decode_noalloc(float* out, const float* q_gate, const float* k,
                                              const float* v, uint16_t* k_cache, uint16_t* v_cache,
                                              const float* q_norm_w, const float* k_norm_w, int n_heads,
                                              int n_kv_heads, int head_dim, int rot_dim, int pos,
                                              float theta, float eps, int rope_mode, int gate,
                                              const float* cos_row, const float* sin_row,
                                              int* cache_start, int* cache_len, int cache_capacity,
                                              void* stream) {
    ANELM_NONNULL(cache_len);
    ANELM_REQUIRE(n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0,
                  "n_heads %d must be a positive multiple of n_kv_heads %d", n_heads, n_kv_heads);
    ANELM_REQUIRE(cache_capacity > 0, "capacity %d", cache_capacity);
    const int len = *cache_len < cache_capacity ? *cache_len + 1 : cache_capacity;
    const size_t need = full_attn_part_bytes(n_heads, n_kv_heads, head_dim, len);
    if (need > kScratchBytes)
        return set_error(ANELM_ERANGE,
                         "full_attn_decode_noalloc: %d keys need %zu bytes of split partials, the static scratch "
                         "holds %zu", len, need, kScratchBytes);
    float* part = scratch_ptr();
    if (part == nullptr) return ANELM_EHIP;
    return full_attn_decode_impl(out, q_gate, k, v, k_cache, v_cache, q_norm_w, k_norm_w, n_heads, n_kv_heads,
                                 head_dim, rot_dim, pos, theta, eps, rope_mode, gate, cos_row, sin_row,
                                 cache_start, cache_len, cache_capacity, as_stream(stream), part, kScratchBytes);
}

