/*
 * swiftllm_ceilings.h — C ABI of libswiftllm_ceilings.so: measurement
 * kernels that give the decode path's roofline denominators on the box they
 * run on. They have no counterpart in the reference (whose benchmark is a
 * TODO, crates/swiftllm-server/src/main.rs:229-244) and are not part of the
 * drop-in interface (include/swiftllm_hip.h): bench.py times them beside the
 * kernels they bound, on the same inputs.
 *
 * Each kernel repeats one memory access pattern of the path and nothing
 * else (the values it reads are only folded into a word that is stored when
 * it equals a fixed constant, so no load can be removed):
 *   read stream    sequential 16-byte nontemporal loads over a buffer;
 *   tile gather    the K and V tiles of every (sequence, kv head, valid
 *                  block) of a decode batch, through its block tables, with
 *                  8- or 16-byte nontemporal loads (the decode's reads);
 *   cache store    the reshape_and_cache stores of a batch of tokens, 2 bytes
 *                  into each 32-byte row of each touched tile, without the
 *                  loads (or, for comparison, whole 32-byte rows);
 *   row copy       the MoE permute's copies: each row read once and written
 *                  to top_k destination rows with nontemporal stores;
 *   mfma stream    the expert GEMM's matrix instructions alone (its grid,
 *                  waves per SIMD, wave tile and MFMA form) on random fp16
 *                  operands held in registers: the dense fp16 rate this
 *                  box sustains at the clock that much matrix work allows.
 *
 * Return values: 0 on success, -4 for invalid arguments, -6 for unsupported
 * shapes, -2 when the launch fails (the codes of include/swiftllm_hip.h).
 * All pointers are device memory; launches are asynchronous on `stream`.
 */
#ifndef SWIFTLLM_CEILINGS_H
#define SWIFTLLM_CEILINGS_H

#include <stddef.h>
#include <stdint.h>

#if defined(__has_include)
#if __has_include(<hip/hip_runtime_api.h>)
#include <hip/hip_runtime_api.h>
#define SWIFTLLM_CEILINGS_HAVE_RUNTIME_API 1
#endif
#endif
#ifndef SWIFTLLM_CEILINGS_HAVE_RUNTIME_API
typedef struct ihipStream_t* hipStream_t;
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* Reads `bytes` bytes at `src` (16-byte aligned, bytes % 16 == 0) once, in
 * 16-byte nontemporal loads; `sink` is a 4-byte device word. */
int swiftllm_ceil_read_stream(const void* src, size_t bytes, uint32_t* sink,
                              hipStream_t stream);

/* Reads the K and V tiles a decode of this batch reads, in the work items
 * of the decode's own decomposition: item i = items[3i .. 3i+2] =
 * (unit = s * num_kv_heads + h, first block, end block) reads the tiles of
 * kv head h at block_tables[s, first .. end - 1] (end clipped to
 * max_num_blocks_per_seq). One 4-wave workgroup per item, in item order,
 * waves taking blocks round-robin, two blocks per wave in flight.
 * load_bytes 8 or 16; head_dim 64 or 128. Items whose unit is negative or
 * names a sequence s >= num_seqs (rows of block_tables) read nothing;
 * block ids outside [0, num_blocks) are skipped (num_blocks <= 0: no
 * bound). */
int swiftllm_ceil_tile_gather(const void* key_cache, const void* value_cache,
                              const int32_t* block_tables, const int32_t* items,
                              int num_items, int num_seqs, int num_kv_heads, int head_dim,
                              int max_num_blocks_per_seq, int num_blocks,
                              int load_bytes, uint32_t* sink,
                              hipStream_t stream);

/* The stores of reshape_and_cache for num_tokens tokens at slot_mapping
 * (negative slots and slots past num_blocks * 16 skipped), writing a
 * per-token constant instead of loaded
 * values. mode 0: each thread stores 4 consecutive d rows of a head with
 * four 2-byte stores; mode 1: consecutive lanes store consecutive d rows
 * (one 128-byte line per 4 lanes); mode 2: each touched 32-byte row written
 * whole by two 16-byte stores (not the cache write's semantics: the
 * layout's full-row store rate, for comparison). */
int swiftllm_ceil_cache_store(void* key_cache, void* value_cache,
                              const int32_t* slot_mapping, int num_tokens,
                              int num_kv_heads, int head_dim, int num_blocks,
                              int mode, hipStream_t stream);

/* dst[dst_rows[t * top_k + k], :] = src[t, :] for every token t and k <
 * top_k (rows of `hidden` fp16, hidden % 512 == 0, 16-byte aligned rows);
 * entries outside [0, num_dst_rows) are not written. */
int swiftllm_ceil_row_copy(const void* src, void* dst, const int32_t* dst_rows,
                           int num_tokens, int top_k, int hidden,
                           int num_dst_rows, hipStream_t stream);

/* num_groups workgroups of 8 waves, each wave issuing `stages` x 32
 * v_mfma_f32_32x32x16_f16 (4 k steps of a 128 x 64 tile per 64-k stage:
 * 2 * 32 * 32 * 16 * 32 FLOP per wave per stage) on operands read once from
 * `operands` (operand_bytes >= 1024, 16-byte aligned; fill it with random
 * fp16 like the GEMM's data). */
int swiftllm_ceil_mfma_stream(const void* operands, size_t operand_bytes,
                              int num_groups, int stages, uint32_t* sink,
                              hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* SWIFTLLM_CEILINGS_H */
