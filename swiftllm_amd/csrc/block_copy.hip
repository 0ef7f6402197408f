// Block copies of the paged KV cache for gfx950: copy_blocks (copy-on-write
// inside the device pool) and swap_blocks (between the device pool and a
// pinned host pool).
//
// Contract. block_mapping holds num_pairs (src, dst) pairs of int64 block
// ids. For every pair and every cache array, the block's bytes move from src
// to dst:
//   copy_blocks (paged_attention.cu:201-227, launcher cu:302-327, and the
//   layered form of crates/swiftllm-cuda/src/bindings.rs:201-223):
//     K_l[dst] = K_l[src], V_l[dst] = V_l[src] for every layer l, where a
//     block of the [NB, Hkv, D, BS] layout is Hkv*D*BS contiguous fp16.
//   swap_blocks (bindings.rs:225-242): dst[dst_id*bytes ..][0..bytes) =
//     src[src_id*bytes ..][0..bytes) for a block of block_size_bytes.
// A pair with a negative id is skipped (padding), and so is a pair with an id
// past a known pool size. Destinations must be distinct and must not be the
// source of another pair in the same call (otherwise the result is
// unspecified, as in the reference's parallel kernel).
//
// The reference kernel launches head_dim * block_size threads per workgroup
// (2048 at D 128, BS 16), past the 1024-thread limit, so its launch fails.
// Here one kernel moves every (pair, array, chunk) in one launch: a
// workgroup moves a chunk of about 16 KiB with 16-byte accesses, four loads
// per thread in flight before the stores. Loads and stores are nontemporal:
// each byte is read once and the copy is not read back by this kernel.
// Pinned host memory is addressed directly by the kernel, so a swap in
// either direction is one launch instead of one DMA request per block.

#include "common.hpp"

namespace swiftllm {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int kCopyThreads = 256;
constexpr int kCopyUnroll = 4;
constexpr int kMaxCopyArrays = 64;              // arrays per launch (larger sets loop)
constexpr size_t kChunkBytes = 16384;           // bytes per workgroup

struct BlockCopyArgs {
    const long long* mapping;  // [pairs][2]: src, dst
    long long src_blocks;      // bound on src ids; <= 0: unbounded
    long long dst_blocks;      // bound on dst ids; <= 0: unbounded
    size_t block_bytes;
    int chunks;                // workgroups per (pair, array)
    int vec;                   // 1: 16-byte path
    const char* src[kMaxCopyArrays];
    char* dst[kMaxCopyArrays];
};

__global__ __launch_bounds__(kCopyThreads) void block_copy_kernel(const BlockCopyArgs a) {
    const int pair = blockIdx.x / a.chunks;
    const int chunk = blockIdx.x - pair * a.chunks;
    const int arr = blockIdx.y;
    const long long s = a.mapping[2 * static_cast<size_t>(pair)];
    const long long d = a.mapping[2 * static_cast<size_t>(pair) + 1];
    if (s < 0 || d < 0 || (a.src_blocks > 0 && s >= a.src_blocks) ||
        (a.dst_blocks > 0 && d >= a.dst_blocks)) {
        return;
    }
    const char* src = a.src[arr] + static_cast<size_t>(s) * a.block_bytes;
    char* dst = a.dst[arr] + static_cast<size_t>(d) * a.block_bytes;
    if (a.vec) {
        const size_t nv = a.block_bytes / 16;
        const size_t per = (nv + a.chunks - 1) / a.chunks;
        const size_t v0 = static_cast<size_t>(chunk) * per;
        const size_t v1 = v0 + per < nv ? v0 + per : nv;
        const u32x4* __restrict__ sv = reinterpret_cast<const u32x4*>(src);
        u32x4* __restrict__ dv = reinterpret_cast<u32x4*>(dst);
        for (size_t i0 = v0 + threadIdx.x; i0 < v1; i0 += kCopyThreads * kCopyUnroll) {
            u32x4 v[kCopyUnroll];
#pragma unroll
            for (int u = 0; u < kCopyUnroll; ++u) {
                const size_t i = i0 + static_cast<size_t>(u) * kCopyThreads;
                if (i < v1) v[u] = __builtin_nontemporal_load(sv + i);
            }
#pragma unroll
            for (int u = 0; u < kCopyUnroll; ++u) {
                const size_t i = i0 + static_cast<size_t>(u) * kCopyThreads;
                if (i < v1) __builtin_nontemporal_store(v[u], dv + i);
            }
        }
    } else {
        const size_t per = (a.block_bytes + a.chunks - 1) / a.chunks;
        const size_t b0 = static_cast<size_t>(chunk) * per;
        const size_t b1 = b0 + per < a.block_bytes ? b0 + per : a.block_bytes;
        for (size_t i = b0 + threadIdx.x; i < b1; i += kCopyThreads) dst[i] = src[i];
    }
}

// Moves the mapped blocks of `n` arrays (src[i] -> dst[i]).
int copy_arrays(const char* who, const long long* mapping, long long num_pairs,
                const char* const* src, char* const* dst, long long n, size_t block_bytes,
                long long src_blocks, long long dst_blocks, hipStream_t stream) {
    if (num_pairs < 0 || n < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_pairs=%lld arrays=%lld", who,
                    num_pairs, n);
    }
    if (num_pairs > 0 && n > 0 && (mapping == nullptr || block_bytes == 0)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null mapping or empty blocks", who);
    }
    if (!aligned(mapping, 8)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: misaligned block_mapping", who);
    }
    const size_t chunks_ll = (block_bytes + kChunkBytes - 1) / kChunkBytes;
    if (num_pairs > 0 && static_cast<unsigned long long>(num_pairs) * (chunks_ll ? chunks_ll : 1) >
                             0x7fffffffULL) {
        return fail(SWIFTLLM_ERR_NOT_SUPPORTED, "%s: %lld pairs of %zu bytes is too many for one launch",
                    who, num_pairs, block_bytes);
    }
    bool vec = block_bytes % 16 == 0;
    for (long long i = 0; i < n; ++i) {
        if (num_pairs > 0 && (src[i] == nullptr || dst[i] == nullptr)) {
            return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null cache pointer (array %lld)", who, i);
        }
        vec = vec && aligned(src[i], 16) && aligned(dst[i], 16);
    }
    int rc = require_device();
    if (rc != SWIFTLLM_OK) return rc;
    if (num_pairs == 0 || n == 0) return ok();
    BlockCopyArgs a{};
    a.mapping = mapping;
    a.src_blocks = src_blocks;
    a.dst_blocks = dst_blocks;
    a.block_bytes = block_bytes;
    a.chunks = static_cast<int>(chunks_ll ? chunks_ll : 1);
    a.vec = vec ? 1 : 0;
    for (long long base = 0; base < n; base += kMaxCopyArrays) {
        const int m = static_cast<int>(n - base < kMaxCopyArrays ? n - base : kMaxCopyArrays);
        for (int i = 0; i < m; ++i) {
            a.src[i] = src[base + i];
            a.dst[i] = dst[base + i];
        }
        const dim3 grid(static_cast<unsigned>(num_pairs * a.chunks), static_cast<unsigned>(m));
        hipError_t err = launch(block_copy_kernel, grid, dim3(kCopyThreads), 0, stream, a);
        if (err != hipSuccess) return launched(err, who);
    }
    return ok();
}

int copy_blocks(const char* who, const int64_t* mapping, long long num_pairs,
                void* const* key_caches, void* const* value_caches, long long num_layers,
                long long num_kv_heads, long long head_dim, long long block_size,
                long long num_blocks, hipStream_t stream) {
    if (num_layers < 0 || num_kv_heads <= 0 || head_dim <= 0 || block_size <= 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER,
                    "%s: num_layers=%lld num_kv_heads=%lld head_dim=%lld block_size=%lld", who,
                    num_layers, num_kv_heads, head_dim, block_size);
    }
    if (num_layers > 0 && (key_caches == nullptr || value_caches == nullptr)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: null cache list", who);
    }
    const unsigned long long elems = static_cast<unsigned long long>(num_kv_heads) * head_dim *
                                     block_size;
    if (elems > (1ULL << 40)) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: block of %llu elements", who, elems);
    }
    if (num_pairs < 0) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_pairs=%lld", who, num_pairs);
    }
    if (num_layers == 0) {
        const int rc = require_device();
        return rc != SWIFTLLM_OK ? rc : ok();
    }
    // Per launch, the K caches of up to kMaxCopyArrays / 2 layers, then their V caches.
    constexpr long long kLayers = kMaxCopyArrays / 2;
    const char* src[kMaxCopyArrays];
    char* dst[kMaxCopyArrays];
    for (long long base = 0; base < num_layers; base += kLayers) {
        const long long m = num_layers - base < kLayers ? num_layers - base : kLayers;
        for (long long i = 0; i < m; ++i) {
            src[i] = dst[i] = static_cast<char*>(key_caches[base + i]);
            src[m + i] = dst[m + i] = static_cast<char*>(value_caches[base + i]);
        }
        const int rc = copy_arrays(who, reinterpret_cast<const long long*>(mapping), num_pairs, src,
                                   dst, 2 * m, elems * 2, num_blocks, num_blocks, stream);
        if (rc != SWIFTLLM_OK) return rc;
    }
    return ok();
}

}  // namespace
}  // namespace swiftllm

using namespace swiftllm;

extern "C" {

void launch_copy_blocks(int64_t* block_mapping, void* key_cache, void* value_cache, int num_pairs,
                        int num_kv_heads, int head_dim, int block_size, hipStream_t stream) {
    void* kc[1] = {key_cache};
    void* vc[1] = {value_cache};
    copy_blocks("launch_copy_blocks", block_mapping, num_pairs, kc, vc, 1, num_kv_heads, head_dim,
                block_size, 0, stream);
}

int swiftllm_hip_launch_copy_blocks(const int64_t* block_mapping, void* key_cache,
                                    void* value_cache, int num_pairs, int num_kv_heads,
                                    int head_dim, int block_size, int num_blocks,
                                    hipStream_t stream) {
    void* kc[1] = {key_cache};
    void* vc[1] = {value_cache};
    return copy_blocks("swiftllm_hip_launch_copy_blocks", block_mapping, num_pairs, kc, vc, 1,
                       num_kv_heads, head_dim, block_size, num_blocks, stream);
}

int swiftllm_hip_copy_blocks(void* const* key_caches, void* const* value_caches,
                             const int64_t* block_mapping, size_t num_pairs, size_t num_layers,
                             size_t num_kv_heads, size_t head_dim, size_t block_size,
                             hipStream_t stream) {
    const char* who = "swiftllm_hip_copy_blocks";
    const size_t lim = 0x7fffffff;
    if (num_pairs > lim || num_layers > lim || num_kv_heads > lim || head_dim > lim ||
        block_size > lim) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: parameter out of range", who);
    }
    return copy_blocks(who, block_mapping, static_cast<long long>(num_pairs), key_caches,
                       value_caches, static_cast<long long>(num_layers),
                       static_cast<long long>(num_kv_heads), static_cast<long long>(head_dim),
                       static_cast<long long>(block_size), 0, stream);
}

int swiftllm_hip_swap_blocks(const void* src, void* dst, const int64_t* block_mapping,
                             size_t num_pairs, size_t block_size_bytes, hipStream_t stream) {
    const char* who = "swiftllm_hip_swap_blocks";
    if (num_pairs > 0x7fffffff) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_pairs out of range", who);
    }
    const char* s[1] = {static_cast<const char*>(src)};
    char* d[1] = {static_cast<char*>(dst)};
    return copy_arrays(who, reinterpret_cast<const long long*>(block_mapping),
                       static_cast<long long>(num_pairs), s, d, 1, block_size_bytes, 0, 0, stream);
}

int swiftllm_hip_launch_swap_blocks(const void* src, void* dst, const int64_t* block_mapping,
                                    size_t num_pairs, size_t block_size_bytes, long long src_blocks,
                                    long long dst_blocks, hipStream_t stream) {
    const char* who = "swiftllm_hip_launch_swap_blocks";
    if (num_pairs > 0x7fffffff) {
        return fail(SWIFTLLM_ERR_INVALID_PARAMETER, "%s: num_pairs out of range", who);
    }
    const char* s[1] = {static_cast<const char*>(src)};
    char* d[1] = {static_cast<char*>(dst)};
    return copy_arrays(who, reinterpret_cast<const long long*>(block_mapping),
                       static_cast<long long>(num_pairs), s, d, 1, block_size_bytes, src_blocks,
                       dst_blocks, stream);
}

}  // extern "C"
