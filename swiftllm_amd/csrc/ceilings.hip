// Measurement kernels for gfx950: one memory access pattern each, nothing
// else, so that the time of the pattern alone bounds the path's kernels
// that contain it (include/swiftllm_ceilings.h). Built into its own library,
// libswiftllm_ceilings.so; the drop-in library does not contain them.
//
// Every load feeds an XOR fold whose result is stored only when it equals a
// fixed constant, so the compiler keeps every load and the kernels write
// (almost) nothing but what the pattern itself writes. The one compute
// pattern, the MFMA stream, folds its accumulators the same way.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <type_traits>

#include "swiftllm_ceilings.h"

namespace swiftllm_ceilings {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

constexpr int kOk = 0;
constexpr int kErrKernel = -2;
constexpr int kErrInvalid = -4;
constexpr int kErrUnsupported = -6;
constexpr uint32_t kSinkMagic = 0x9E3779B9u;

__device__ __forceinline__ uint32_t fold(u32x4 v) { return v.x ^ v.y ^ v.z ^ v.w; }
__device__ __forceinline__ uint32_t fold(u32x2 v) { return v.x ^ v.y; }

__device__ __forceinline__ void sink_if(uint32_t x, uint32_t* sink) {
    if (x == kSinkMagic) *sink = x;
}

// Block tables and slots do not change during a kernel; through the
// constant address space wave-uniform reads of them become scalar loads.
typedef __attribute__((address_space(4))) const int const_int;
__device__ __forceinline__ const const_int* as_const(const int* p) {
    return (const const_int*)(p);
}

template <typename Args>
int launch(void (*kernel)(Args), dim3 grid, dim3 block, hipStream_t stream, const Args& args) {
    void* argv[] = {const_cast<Args*>(&args)};
    const hipError_t err =
        hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, argv, 0, stream);
    return err == hipSuccess ? kOk : kErrKernel;
}

bool aligned(const void* p, size_t n) { return reinterpret_cast<uintptr_t>(p) % n == 0; }

int device_cus() {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        return 256;
    }
    return n;
}

// ---------------------------------------------------------------------------
// Sequential read stream: each workgroup reads contiguous chunks of
// 256 x 4 x 16 bytes (four nontemporal loads per thread in flight), chunks
// dealt out grid-stride. Measured on MI355X over a 2 GiB buffer: 7.06-7.36
// TB/s for 4 or 8 loads per thread and 2-32 workgroups per CU, the best at
// 4 loads and 2 workgroups per CU; cached loads 6.2-6.5 TB/s, and a
// grid-stride walk of single 16-byte pieces 5.98 TB/s.
// ---------------------------------------------------------------------------
constexpr int kStreamUnroll = 4;
constexpr int kStreamGroupsPerCU = 2;

struct StreamArgs {
    const u32x4* src;
    long long n16;
    uint32_t* sink;
};

__global__ __launch_bounds__(256) void read_stream_kernel(const StreamArgs a) {
    constexpr long long kChunk = 256LL * kStreamUnroll;
    uint32_t acc = 0;
    for (long long c = static_cast<long long>(blockIdx.x) * kChunk; c < a.n16;
         c += static_cast<long long>(gridDim.x) * kChunk) {
        u32x4 v[kStreamUnroll];
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) {
            const long long i = c + u * 256 + threadIdx.x;
            v[u] = i < a.n16 ? __builtin_nontemporal_load(a.src + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < kStreamUnroll; ++u) acc ^= fold(v[u]);
    }
    sink_if(acc, a.sink);
}

// ---------------------------------------------------------------------------
// Tile gather: the decode's K/V reads. One 4-wave workgroup per item
// (unit = s * Hkv + h, first block, end block) of a block range of one
// sequence and kv head; wave w takes blocks first + w, first + w + 4, ...
// with two blocks' K and V loads in flight (blocks j and j + 4). Whole tiles
// are read, as the decode reads the tail block's tile whole.
// ---------------------------------------------------------------------------
struct GatherArgs {
    const char* kc;
    const char* vc;
    const int* bt;
    const int* items;  // [n][3]
    uint32_t* sink;
    int S;
    int Hkv;
    int MB;
    int num_blocks;
};

template <int D, int LB>
__global__ __launch_bounds__(256) void tile_gather_kernel(const GatherArgs a) {
    using V = typename std::conditional<LB == 16, u32x4, u32x2>::type;
    constexpr int N = D / 2 / LB;                          // loads per lane per tile
    constexpr size_t kTile = static_cast<size_t>(D) * 32;  // bytes per tile
    const const_int* item = as_const(a.items) + 3 * static_cast<size_t>(blockIdx.x);
    const int unit = item[0];
    const int s = unit / a.Hkv;
    const int h = unit - s * a.Hkv;
    if (unit < 0 || s >= a.S) return;  // no row of the block table
    const int first = max(item[1], 0);
    const int end = min(item[2], a.MB);
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int lane = threadIdx.x % 64;
    const const_int* row = as_const(a.bt) + static_cast<size_t>(s) * a.MB;
    auto ok = [&](int b) { return b >= 0 && (a.num_blocks <= 0 || b < a.num_blocks); };
    uint32_t acc = 0;
    for (int j = first + w; j < end; j += 8) {
        const int b0 = row[j];
        const int b1 = (j + 4 < end) ? row[j + 4] : -1;
        V k0[N], v0[N], k1[N], v1[N];
        if (ok(b0)) {
            const size_t base = (static_cast<size_t>(b0) * a.Hkv + h) * kTile + lane * LB;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                k0[i] = __builtin_nontemporal_load(reinterpret_cast<const V*>(a.kc + base + i * 64 * LB));
                v0[i] = __builtin_nontemporal_load(reinterpret_cast<const V*>(a.vc + base + i * 64 * LB));
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) k0[i] = v0[i] = V{};
        }
        if (ok(b1)) {
            const size_t base = (static_cast<size_t>(b1) * a.Hkv + h) * kTile + lane * LB;
#pragma unroll
            for (int i = 0; i < N; ++i) {
                k1[i] = __builtin_nontemporal_load(reinterpret_cast<const V*>(a.kc + base + i * 64 * LB));
                v1[i] = __builtin_nontemporal_load(reinterpret_cast<const V*>(a.vc + base + i * 64 * LB));
            }
        } else {
#pragma unroll
            for (int i = 0; i < N; ++i) k1[i] = v1[i] = V{};
        }
#pragma unroll
        for (int i = 0; i < N; ++i) acc ^= fold(k0[i]) ^ fold(v0[i]) ^ fold(k1[i]) ^ fold(v1[i]);
    }
    sink_if(acc, a.sink);
}

// ---------------------------------------------------------------------------
// Cache-write stores: 2 bytes into each of the Hkv * D rows of the token's
// block (row r = h * D + d of block b at element (b * Hkv * D + r) * 16),
// at column o = slot % 16, for K and for V.
// ---------------------------------------------------------------------------
struct StoreArgs {
    uint16_t* kc;
    uint16_t* vc;
    const int* slots;
    long long num_slots;
    int rows;  // Hkv * D
};

template <int MODE>
__global__ __launch_bounds__(256) void cache_store_kernel(const StoreArgs a) {
    const int t = blockIdx.x;
    const int slot = a.slots[t];
    if (slot < 0 || (a.num_slots > 0 && slot >= a.num_slots)) return;
    const int b = slot >> 4;
    const int o = slot & 15;
    const size_t blk = static_cast<size_t>(b) * a.rows * 16;
    const uint16_t val = static_cast<uint16_t>((t * 2654435761u) >> 16);
    if constexpr (MODE == 0) {
        for (int r = threadIdx.x * 4; r < a.rows; r += 1024) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                __builtin_nontemporal_store(val, a.kc + blk + static_cast<size_t>(r + i) * 16 + o);
                __builtin_nontemporal_store(val, a.vc + blk + static_cast<size_t>(r + i) * 16 + o);
            }
        }
    } else if constexpr (MODE == 1) {
        for (int r = threadIdx.x; r < a.rows; r += 256) {
            __builtin_nontemporal_store(val, a.kc + blk + static_cast<size_t>(r) * 16 + o);
            __builtin_nontemporal_store(val, a.vc + blk + static_cast<size_t>(r) * 16 + o);
        }
    } else {
        const u32x4 v = {val, val, val, val};
        for (int i = threadIdx.x; i < 2 * a.rows; i += 256) {
            const size_t e = blk + static_cast<size_t>(i >> 1) * 16 + (i & 1) * 8;
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.kc + e));
            __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(a.vc + e));
        }
    }
}

// ---------------------------------------------------------------------------
// Row copy: one wave per token reads its row (8 KiB at hidden 4096: eight
// 16-byte loads per lane in flight) and stores it to top_k rows.
// ---------------------------------------------------------------------------
struct CopyArgs {
    const u32x4* src;
    u32x4* dst;
    const int* rows;
    int T;
    int K;
    int n16;  // 16-byte pieces per row
    int num_dst_rows;
};

__global__ __launch_bounds__(256) void row_copy_kernel(const CopyArgs a) {
    const int t = blockIdx.x * 4 + threadIdx.x / 64;
    if (t >= a.T) return;
    const int lane = threadIdx.x % 64;
    const int per = a.n16 / 64;
    for (int c0 = 0; c0 < per; c0 += 8) {
        const int cnt = min(8, per - c0);
        u32x4 v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (i < cnt) {
                v[i] = __builtin_nontemporal_load(a.src + static_cast<size_t>(t) * a.n16 + (c0 + i) * 64 + lane);
            }
        }
        for (int k = 0; k < a.K; ++k) {
            const int r = a.rows[t * a.K + k];
            if (r < 0 || r >= a.num_dst_rows) continue;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                if (i < cnt) {
                    __builtin_nontemporal_store(v[i], a.dst + static_cast<size_t>(r) * a.n16 + (c0 + i) * 64 + lane);
                }
            }
        }
    }
}

// MFMA stream: the expert GEMM's matrix work with no memory traffic in the
// loop. Workgroups of 8 waves (two per SIMD, the GEMM's occupancy); per
// 64-k stage each wave issues 4 k steps of 8 v_mfma_f32_32x32x16_f16 into
// 8 accumulators (the GEMM's 128 x 64 wave tile). The 4 steps use 4
// different operand sets, loaded once from random fp16 the caller provides,
// so successive MFMAs see different data as they do in the GEMM: the
// matrix cores' power, and so the clock they sustain, depends on the data
// (constant operands run faster than random ones).
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f16x __attribute__((ext_vector_type(16)));
constexpr int kMfmaWaves = 8;
constexpr int kMfmaSteps = 4;  // k steps of 16 per 64-k stage
constexpr float kMfmaSinkValue = 1.2345678e30f;

struct MfmaArgs {
    const h8* ops;  // n_ops fragments of 64 lanes x 8 halves
    uint32_t* sink;
    int n_ops;
    int stages;
};

__global__ __launch_bounds__(64 * kMfmaWaves) void mfma_stream_kernel(const MfmaArgs a) {
    const int lane = threadIdx.x % 64;
    const int wv = threadIdx.x / 64;
    const long long base = (static_cast<long long>(blockIdx.x) * kMfmaWaves + wv) * kMfmaSteps * 6;
    h8 x[kMfmaSteps][4], w[kMfmaSteps][2];
#pragma unroll
    for (int s = 0; s < kMfmaSteps; ++s) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            x[s][j] = a.ops[((base + s * 6 + j) % a.n_ops) * 64 + lane];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            w[s][i] = a.ops[((base + s * 6 + 4 + i) % a.n_ops) * 64 + lane];
        }
    }
    f16x acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f16x{};
    for (int st = 0; st < a.stages; ++st) {
#pragma unroll
        for (int s = 0; s < kMfmaSteps; ++s)
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(w[s][i], x[s][j], acc[i][j], 0, 0, 0);
    }
    // A float sum: hipcc (ROCm 7.2) drops the whole kernel when the
    // accumulators are folded by their bit patterns instead.
    float f = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) f += acc[i][j][r];
    if (f == kMfmaSinkValue) *a.sink = kSinkMagic;
}

}  // namespace
}  // namespace swiftllm_ceilings

using namespace swiftllm_ceilings;

extern "C" {

int swiftllm_ceil_read_stream(const void* src, size_t bytes, uint32_t* sink, hipStream_t stream) {
    if (!src || !sink || !aligned(src, 16) || bytes % 16 != 0) return kErrInvalid;
    if (bytes == 0) return kOk;
    StreamArgs a{static_cast<const u32x4*>(src), static_cast<long long>(bytes / 16), sink};
    const long long chunks = (a.n16 + 256LL * kStreamUnroll - 1) / (256LL * kStreamUnroll);
    const long long groups = std::min<long long>(chunks, 1LL * kStreamGroupsPerCU * device_cus());
    return launch(read_stream_kernel, dim3(static_cast<unsigned>(groups)), dim3(256), stream, a);
}

int swiftllm_ceil_tile_gather(const void* key_cache, const void* value_cache,
                              const int32_t* block_tables, const int32_t* items, int num_items,
                              int num_seqs, int num_kv_heads, int head_dim, int max_num_blocks_per_seq,
                              int num_blocks, int load_bytes, uint32_t* sink, hipStream_t stream) {
    if (num_items < 0 || num_seqs < 0 || num_kv_heads <= 0 || max_num_blocks_per_seq < 0) {
        return kErrInvalid;
    }
    if ((head_dim != 64 && head_dim != 128) || (load_bytes != 8 && load_bytes != 16)) {
        return kErrUnsupported;
    }
    if (num_items == 0) return kOk;
    if (!key_cache || !value_cache || !block_tables || !items || !sink ||
        !aligned(key_cache, load_bytes) || !aligned(value_cache, load_bytes)) {
        return kErrInvalid;
    }
    GatherArgs a{static_cast<const char*>(key_cache), static_cast<const char*>(value_cache),
                 block_tables, items, sink, num_seqs, num_kv_heads, max_num_blocks_per_seq, num_blocks};
    auto k = head_dim == 128 ? (load_bytes == 16 ? tile_gather_kernel<128, 16> : tile_gather_kernel<128, 8>)
                             : (load_bytes == 16 ? tile_gather_kernel<64, 16> : tile_gather_kernel<64, 8>);
    return launch(k, dim3(num_items), dim3(256), stream, a);
}

int swiftllm_ceil_cache_store(void* key_cache, void* value_cache, const int32_t* slot_mapping,
                              int num_tokens, int num_kv_heads, int head_dim, int num_blocks,
                              int mode, hipStream_t stream) {
    if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || mode < 0 || mode > 2) {
        return kErrInvalid;
    }
    if (head_dim % 4 != 0) return kErrUnsupported;
    if (num_tokens == 0) return kOk;
    if (!key_cache || !value_cache || !slot_mapping || !aligned(key_cache, 32) ||
        !aligned(value_cache, 32)) {
        return kErrInvalid;
    }
    StoreArgs a{static_cast<uint16_t*>(key_cache), static_cast<uint16_t*>(value_cache), slot_mapping,
                num_blocks > 0 ? static_cast<long long>(num_blocks) * 16 : 0, num_kv_heads * head_dim};
    auto k = mode == 0 ? cache_store_kernel<0> : mode == 1 ? cache_store_kernel<1> : cache_store_kernel<2>;
    return launch(k, dim3(num_tokens), dim3(256), stream, a);
}

int swiftllm_ceil_row_copy(const void* src, void* dst, const int32_t* dst_rows, int num_tokens,
                           int top_k, int hidden, int num_dst_rows, hipStream_t stream) {
    if (num_tokens < 0 || top_k <= 0 || hidden <= 0 || num_dst_rows < 0) return kErrInvalid;
    if (hidden % 512 != 0) return kErrUnsupported;
    if (num_tokens == 0) return kOk;
    if (!src || !dst || !dst_rows || !aligned(src, 16) || !aligned(dst, 16)) return kErrInvalid;
    CopyArgs a{static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), dst_rows, num_tokens, top_k,
               hidden / 8, num_dst_rows};
    return launch(row_copy_kernel, dim3((num_tokens + 3) / 4), dim3(256), stream, a);
}

int swiftllm_ceil_mfma_stream(const void* operands, size_t operand_bytes, int num_groups,
                              int stages, uint32_t* sink, hipStream_t stream) {
    if (num_groups < 0 || stages < 0 || !operands || !sink || !aligned(operands, 16)) return kErrInvalid;
    const long long n_ops = static_cast<long long>(operand_bytes / (64 * sizeof(h8)));
    if (n_ops < 1 || n_ops > 0x7fffffffLL) return kErrInvalid;
    if (num_groups == 0 || stages == 0) return kOk;
    MfmaArgs a{static_cast<const h8*>(operands), sink, static_cast<int>(n_ops), stages};
    return launch(mfma_stream_kernel, dim3(num_groups), dim3(64 * kMfmaWaves), stream, a);
}

}  // extern "C"
