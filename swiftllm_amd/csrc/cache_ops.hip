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
// One workgroup per token, consecutive lanes on consecutive rows. Row
// r = h * D + d of block b is the 16 tokens of (h, d) at element
// (b * Hkv * D + r) * BS; the token's element goes to column o of it. Four
// rows make a 128-byte line (BS 16), so one wave store instruction covers 16
// whole lines with 8 bytes each, where a lane per 4 consecutive d (four
// stores to the 4 rows of one line) needs 64 lines per instruction and four
// instructions per line. Measured alone on MI355X (the stores of config 4's
// 256 tokens, no loads): 8.7 us against 23.4 us.

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

// Rows per thread per pass: a pass of 256 threads covers 1024 rows, all of
// Llama-3-8B's Hkv * D; its 8 loads per thread are issued before any store.
constexpr int kRowsPerThread = 4;

__global__ __launch_bounds__(256) void reshape_and_cache_kernel(const CacheArgs a) {
    const int t = blockIdx.x;
    const int slot = a.slots[t];
    if (slot < 0 || (a.num_slots > 0 && slot >= a.num_slots)) return;
    const int b = slot / a.BS;
    const int o = slot - b * a.BS;
    const int n = a.Hkv * a.D;
    const uint16_t* kr = a.key + t * a.key_stride;
    const uint16_t* vr = a.value + t * a.value_stride;
    uint16_t* kdst = a.kc + static_cast<size_t>(b) * n * a.BS + o;
    uint16_t* vdst = a.vc + static_cast<size_t>(b) * n * a.BS + o;
    for (int r0 = 0; r0 < n; r0 += 256 * kRowsPerThread) {
        uint16_t kv[kRowsPerThread], vv[kRowsPerThread];
#pragma unroll
        for (int i = 0; i < kRowsPerThread; ++i) {
            const int r = r0 + i * 256 + threadIdx.x;
            if (r < n) {
                kv[i] = kr[r];
                vv[i] = vr[r];
            }
        }
#pragma unroll
        for (int i = 0; i < kRowsPerThread; ++i) {
            const int r = r0 + i * 256 + threadIdx.x;
            if (r < n) {
                put(kdst + static_cast<size_t>(r) * a.BS, kv[i]);
                put(vdst + static_cast<size_t>(r) * a.BS, vv[i]);
            }
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
    return launched(launch(reshape_and_cache_kernel, dim3(num_tokens), dim3(256), 0, stream, a),
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
