// Shared helpers for the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "swiftllm_hip.h"

namespace swiftllm {

using f16 = _Float16;
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Host-side status reporting (abi.cpp). Every exported entry point ends in
// ok() or fail(); the void launchers leave the result in the thread-local
// slot read by swiftllm_hip_last_error().
// ---------------------------------------------------------------------------
int ok();
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// SWIFTLLM_OK when a HIP device is visible, else SWIFTLLM_ERR_DEVICE_NOT_FOUND.
int require_device();
// Maps the result of hipLaunchKernel to a status.
int launched(hipError_t err, const char* what);

// Block tables and context lengths do not change during a kernel; reading
// them through the constant address space lets the compiler use scalar loads
// for wave-uniform indices even when the kernel stores to global memory in
// the same loop (those stores would otherwise count as possible clobbers).
typedef __attribute__((address_space(4))) const int const_int;

__device__ __forceinline__ const const_int* as_const(const int* p) {
    return (const const_int*)(p);
}

// Direct memory-to-LDS loads through buffer resources (buffer_load ... lds):
// the resource's base and size are wave-uniform, the lane's byte offset 32
// bits. The compiler adds no waits of its own between these loads and LDS
// reads; every kernel that issues them waits for its loads explicitly.
constexpr int kRsrcWord3 = 0x00020000;   // gfx9 buffer resource: raw 32-bit dwords
typedef __attribute__((address_space(3))) void* lds_ptr;
__device__ __forceinline__ lds_ptr to_lds(void* p) { return (lds_ptr)p; }

// Waits until at most N of this wave's memory loads are in flight (loads
// into LDS by buffer_load ... lds are not tracked by the compiler, so their
// waits are explicit). The empty asm statements keep the compiler from
// moving LDS reads above it.
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | (0x7 << 4) | (0xF << 8) | ((N >> 4) << 14));
    asm volatile("" ::: "memory");
}

inline bool aligned(const void* p, size_t bytes) {
    return (reinterpret_cast<uintptr_t>(p) % bytes) == 0;
}

// Launches `kernel(args)` where the kernel takes one by-value argument
// struct; returns the HIP error of the launch itself.
template <typename Args>
hipError_t launch(void (*kernel)(Args), dim3 grid, dim3 block, size_t lds,
                  hipStream_t stream, const Args& args) {
    void* argv[] = {const_cast<Args*>(&args)};
    return hipLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block,
                           argv, lds, stream);
}

// ---------------------------------------------------------------------------
// KV-cache addressing, layout [num_blocks, num_kv_heads, head_dim, 16]
// (paged_attention.cu:39-40, 85-87, 114-116). One (block, kv head) pair is a
// contiguous tile of head_dim rows of 16 tokens.
// ---------------------------------------------------------------------------
constexpr int kBlockTokens = 16;
// slot >> kBlockShift is the block of a slot. The arithmetic shift keeps a
// negative slot (padding) negative, where slot / 16 would truncate -1..-15
// to block 0.
constexpr int kBlockShift = 4;
static_assert((1 << kBlockShift) == kBlockTokens, "block shift");

__host__ __device__ inline size_t kv_tile_offset(int block, int kv_head,
                                                 int num_kv_heads,
                                                 int head_dim) {
    return (static_cast<size_t>(block) * num_kv_heads + kv_head) *
           static_cast<size_t>(head_dim) * kBlockTokens;
}

// Element (d, t) of a tile.
__host__ __device__ inline int kv_elem_offset(int d, int t) {
    return d * kBlockTokens + t;
}

// ---------------------------------------------------------------------------
// Whole-wave reductions (wave64). Every lane ends with the same value; the
// butterfly adds pairs in the same order in every lane.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_inclusive_scan(int x, int lane) {
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d);
        if (lane >= d) x += y;
    }
    return x;
}

}  // namespace swiftllm
