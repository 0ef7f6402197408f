// KV-cache write (reshape_and_cache) for gfx950.
//
// Contract (paged_attention.cu:167-199, launcher cu:271-300): for token t
// with slot = slot_mapping[t], block b = slot / BS and offset o = slot % BS,
//   key_cache[b, h, d, o]   = key[t, h, d]
//   value_cache[b, h, d, o] = value[t, h, d]
// as bit copies. The reference launches one thread per element for
// head_dim 128 / block_size 16 only (cu:286) and would write out of bounds
// for a negative slot; here any block size and head_dim are taken, negative
// slots are skipped (padding tokens), and slots past num_blocks * BS are
// skipped when the pool size is known.
//
// One workgroup per token. Reads of the token's Hkv*D row are contiguous;
// each element lands in a different 2-byte column of the [D][BS] tile, which
// is the layout's price for having contiguous tokens on the decode side.
// At decode sizes the kernel is bound by those partial-row writes (config 4:
// 2 x 256 x 8 x 128 of them in ~21 us), not by bytes.

#include "common.hpp"

namespace swiftllm {
namespace {

struct CacheArgs {
    const uint16_t* key;
    const uint16_t* value;
    uint16_t* kc;
    uint16_t* vc;
    const int* slots;
    long long key_stride;    // elements between consecutive tokens of key
    long long value_stride;  // elements between consecutive tokens of value
    long long num_slots;     // num_blocks * BS, or <= 0 when unknown
    int Hkv;
    int D;
    int BS;
};

// Each store is 2 bytes of a 32-byte tile row, so the memory system merges
// it into the row (a read-modify-write below the caches). Nontemporal stores
// do that inside this kernel. Cached stores leave partly dirty lines that are
// written back while the next kernel (the decode) streams the pool, and
// writes mixed into that read stream cost it more than this kernel's own
// time (config 4: 21 us here and no decode slowdown, against 9 us here and
// 10-17 us added to the decode).
__device__ __forceinline__ void put(uint16_t* p, uint16_t v) {
    __builtin_nontemporal_store(v, p);
}

// VEC: each thread moves 4 consecutive elements of one head (one 8-byte load
// of key and of value; needs D % 4 == 0 and 8-byte aligned rows), so at
// Llama-3-8B's 1024 elements per token every load of a workgroup is issued
// at once.
template <bool VEC>
__global__ __launch_bounds__(256) void reshape_and_cache_kernel(const CacheArgs a) {
    const int t = blockIdx.x;
    const int slot = a.slots[t];
    if (slot < 0 || (a.num_slots > 0 && slot >= a.num_slots)) return;
    const int b = slot / a.BS;
    const int o = slot - b * a.BS;
    const int n = a.Hkv * a.D;
    const uint16_t* kr = a.key + t * a.key_stride;
    const uint16_t* vr = a.value + t * a.value_stride;
    const size_t tile = static_cast<size_t>(a.D) * a.BS;
    const size_t blk = static_cast<size_t>(b) * a.Hkv * tile + o;
    if constexpr (VEC) {
        for (int e = threadIdx.x * 4; e < n; e += blockDim.x * 4) {
            const uint2 kw = *reinterpret_cast<const uint2*>(kr + e);
            const uint2 vw = *reinterpret_cast<const uint2*>(vr + e);
            const int h = e / a.D;
            const int d = e - h * a.D;
            const size_t dst = blk + h * tile + static_cast<size_t>(d) * a.BS;
            put(a.kc + dst, static_cast<uint16_t>(kw.x));
            put(a.kc + dst + a.BS, static_cast<uint16_t>(kw.x >> 16));
            put(a.kc + dst + 2 * a.BS, static_cast<uint16_t>(kw.y));
            put(a.kc + dst + 3 * a.BS, static_cast<uint16_t>(kw.y >> 16));
            put(a.vc + dst, static_cast<uint16_t>(vw.x));
            put(a.vc + dst + a.BS, static_cast<uint16_t>(vw.x >> 16));
            put(a.vc + dst + 2 * a.BS, static_cast<uint16_t>(vw.y));
            put(a.vc + dst + 3 * a.BS, static_cast<uint16_t>(vw.y >> 16));
        }
    } else {
        for (int e = threadIdx.x; e < n; e += blockDim.x) {
            const int h = e / a.D;
            const int d = e - h * a.D;
            const size_t dst = blk + h * tile + static_cast<size_t>(d) * a.BS;
            put(a.kc + dst, kr[e]);
            put(a.vc + dst, vr[e]);
        }
    }
}

int reshape_and_cache(const void* key, const void* value, void* key_cache, void* value_cache,
                      const int* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                      int block_size, int num_blocks, hipStream_t stream, const char* who) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: num_tokens=%d num_kv_heads=%d head_dim=%d block_size=%d", who, num_tokens,
                    num_kv_heads, head_dim, block_size);
    }
    if (num_tokens > 0 && (!key || !value || !key_cache || !value_cache || !slot_mapping)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null pointer", who);
    }
    if (!aligned(key, 2) || !aligned(value, 2) || !aligned(key_cache, 2) ||
        !aligned(value_cache, 2) || !aligned(slot_mapping, 4)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned pointer", who);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (num_tokens == 0) return ok();
    CacheArgs a{};
    a.key = static_cast<const uint16_t*>(key);
    a.value = static_cast<const uint16_t*>(value);
    a.kc = static_cast<uint16_t*>(key_cache);
    a.vc = static_cast<uint16_t*>(value_cache);
    a.slots = slot_mapping;
    a.key_stride = static_cast<long long>(num_kv_heads) * head_dim;  // cu:294
    a.value_stride = a.key_stride;                                   // cu:295
    a.num_slots = num_blocks > 0 ? static_cast<long long>(num_blocks) * block_size : 0;
    a.Hkv = num_kv_heads;
    a.D = head_dim;
    a.BS = block_size;
    const bool vec = head_dim % 4 == 0 && aligned(key, 8) && aligned(value, 8);
    return launched(launch(vec ? reshape_and_cache_kernel<true> : reshape_and_cache_kernel<false>,
                           dim3(num_tokens), dim3(256), 0, stream, a),
                    who);
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

void launch_reshape_and_cache(void* key, void* value, void* key_cache, void* value_cache,
                              int* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
                              int block_size, hipStream_t stream) {
    reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens, num_kv_heads,
                      head_dim, block_size, 0, stream, "launch_reshape_and_cache");
}

int swiftllm_hip_launch_reshape_and_cache(const void* key, const void* value, void* key_cache,
                                          void* value_cache, const int* slot_mapping,
                                          int num_tokens, int num_kv_heads, int head_dim,
                                          int block_size, int num_blocks, hipStream_t stream) {
    return reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, num_tokens,
                             num_kv_heads, head_dim, block_size, num_blocks, stream,
                             "swiftllm_hip_launch_reshape_and_cache");
}

int swiftllm_hip_reshape_and_cache(const void* key, const void* value, void* key_cache,
                                   void* value_cache, const int32_t* slot_mapping,
                                   const swiftllm_reshape_cache_params* p, hipStream_t stream) {
    const char* who = "swiftllm_hip_reshape_and_cache";
    if (p == nullptr) return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null params", who);
    const size_t lim = 0x7fffffff;
    if (p->num_tokens > lim || p->num_kv_heads > lim || p->head_dim > lim || p->block_size > lim) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: parameter out of range", who);
    }
    return reshape_and_cache(key, value, key_cache, value_cache, slot_mapping,
                             static_cast<int>(p->num_tokens), static_cast<int>(p->num_kv_heads),
                             static_cast<int>(p->head_dim), static_cast<int>(p->block_size), 0,
                             stream, who);
}

}  // extern "C"
