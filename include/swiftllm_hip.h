/*
 * swiftllm_hip.h — C ABI of libswiftllm_hip.so, the MI355X (gfx950) decode
 * hot path: paged-attention decode (single pass and split-K), the
 * reshape_and_cache KV-cache write, and MoE top-k routing / dispatch.
 *
 * Every entry point:
 *   - takes caller-owned device pointers on the current HIP device;
 *   - allocates nothing (scratch memory is passed in by the caller, except
 *     for swiftllm_hip_launch_paged_attention_v2_noalloc, whose scratch is a
 *     static device array);
 *   - is asynchronous on the given stream (NULL = the default stream);
 *   - validates its arguments synchronously on the host before any launch.
 *
 * Device memory layouts (row-major, fp16 = IEEE binary16):
 *   query, output       [num_seqs, num_heads, head_dim]
 *   key/value cache     [num_blocks, num_kv_heads, head_dim, block_size]
 *   block_tables        int32 [num_seqs, max_num_blocks_per_seq]
 *   context_lens        int32 [num_seqs]
 *   key, value (new)    [num_tokens, num_kv_heads, head_dim]
 *   slot_mapping        int32 [num_tokens]; slot = block * block_size + offset
 *
 * Reference interfaces replaced (paths relative to the swiftllm repository):
 *   crates/swiftllm-cuda/kernels/paged_attention.cu:230-327  (extern "C" launchers)
 *   crates/swiftllm-cuda/src/bindings.rs:8-113              (params structs, wrappers)
 *   crates/swiftllm-cuda/src/lib.rs:16-42                   (CudaError variants)
 */
#ifndef SWIFTLLM_HIP_H
#define SWIFTLLM_HIP_H

#include <stddef.h>
#include <stdint.h>

#if defined(__has_include)
#if __has_include(<hip/hip_runtime_api.h>)
#include <hip/hip_runtime_api.h>
#define SWIFTLLM_HIP_HAVE_RUNTIME_API 1
#endif
#endif
#ifndef SWIFTLLM_HIP_HAVE_RUNTIME_API
typedef struct ihipStream_t* hipStream_t;
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------------ */
/* Status codes. Negative values mirror the CudaError variants of            */
/* crates/swiftllm-cuda/src/lib.rs:16-42, in declaration order.              */
/* ------------------------------------------------------------------------ */
typedef enum swiftllm_status {
    SWIFTLLM_OK = 0,
    SWIFTLLM_ERR_INIT = -1,              /* CudaError::InitError        */
    SWIFTLLM_ERR_KERNEL = -2,            /* CudaError::KernelError      */
    SWIFTLLM_ERR_MEMORY = -3,            /* CudaError::MemoryError      */
    SWIFTLLM_ERR_INVALID_PARAMETER = -4, /* CudaError::InvalidParameter */
    SWIFTLLM_ERR_DEVICE_NOT_FOUND = -5,  /* CudaError::DeviceNotFound   */
    SWIFTLLM_ERR_NOT_SUPPORTED = -6      /* CudaError::NotSupported     */
} swiftllm_status;

/* Status of the most recent call made on this host thread (the void
 * launchers report failures only through this), and its message (the
 * String payload of the CudaError variant). The message pointer stays valid
 * until the next call on the same thread. */
int swiftllm_hip_last_error(void);
const char* swiftllm_hip_last_error_message(void);

/* Library version string, e.g. "0.1.0 gfx950". */
const char* swiftllm_hip_version(void);

/* SWIFTLLM_OK when at least one HIP device is visible, else
 * SWIFTLLM_ERR_DEVICE_NOT_FOUND (the no-device behaviour of bindings.rs:72-75). */
int swiftllm_hip_device_check(void);

/* ------------------------------------------------------------------------ */
/* 1. Drop-in launchers: same names and parameter lists as                   */
/*    paged_attention.cu:232-300, with hipStream_t for cudaStream_t.         */
/*    They return void; failures are readable via swiftllm_hip_last_error(). */
/* ------------------------------------------------------------------------ */

/* Replaces launch_paged_attention_v1 (paged_attention.cu:232-269).
 * Single-pass decode: out[s,h] = softmax(scale * q[s,h] . K^T) . V over the
 * first context_lens[s] tokens of sequence s, with kv head h / (H / Hkv).
 * head_dim in {64, 128}; block_size 16; num_heads % num_kv_heads == 0.
 * context_lens[s] <= 0 writes zeros. */
void launch_paged_attention_v1(void* output, void* query, void* key_cache,
                               void* value_cache, int* block_tables,
                               int* context_lens, float scale, int num_seqs,
                               int num_heads, int num_kv_heads, int head_dim,
                               int block_size, int max_num_blocks_per_seq,
                               hipStream_t stream);

/* Replaces launch_reshape_and_cache (paged_attention.cu:271-300).
 * key_cache[slot / bs, h, d, slot % bs] = key[t, h, d] (bit copy), same for
 * value. Tokens with slot_mapping[t] < 0 are skipped (padding). */
void launch_reshape_and_cache(void* key, void* value, void* key_cache,
                              void* value_cache, int* slot_mapping,
                              int num_tokens, int num_kv_heads, int head_dim,
                              int block_size, hipStream_t stream);

/* Split-K decode (the intent of paged_attention_v2_kernel,
 * paged_attention.cu:139-163, whose body is empty and which has no
 * launcher). The context of each sequence is cut into partitions of
 * partition_size tokens (a multiple of 16). A first kernel attends each
 * partition and keeps (max logit, exp sum, partial output) in `workspace`;
 * a second kernel rescales and reduces the partitions of every sequence
 * that has more than one (a sequence with a single partition is written by
 * the first kernel directly). For partitions of up to 1024 tokens and at
 * most a quarter as many sequences as the grid has teams of waves, the
 * first kernel runs as partition streams: every team of waves takes an
 * equal range of the batch's blocks and leaves a partial at each partition
 * end it meets; the workspace then also holds one boundary slot per wave of
 * the grid, which is sized from the current device's compute units (as is
 * the size query's answer).
 * partition_size 0 selects balanced scheduling instead: the blocks of all
 * sequences are split into equal ranges, one per team of waves, so a ragged
 * batch has no long tail; ranges that cut a sequence leave fragments that a
 * second kernel combines. Shapes it cannot take (more than 4096 sequences,
 * or teams so wide that fewer than four fit in the resident grid) fall back
 * to partitions of 512 tokens; the workspace size query covers both.
 * `workspace` holds at least
 * swiftllm_hip_paged_attention_v2_workspace_size() bytes, 256-byte aligned;
 * it is plain scratch (no initialisation, contents unspecified after the
 * call). Calls that share a workspace must be ordered on one stream. */
void launch_paged_attention_v2(void* output, void* workspace,
                               size_t workspace_bytes, void* query,
                               void* key_cache, void* value_cache,
                               int* block_tables, int* context_lens,
                               float scale, int num_seqs, int num_heads,
                               int num_kv_heads, int head_dim, int block_size,
                               int max_num_blocks_per_seq, int partition_size,
                               hipStream_t stream);

/* Bytes of workspace launch_paged_attention_v2 needs for these sizes. */
size_t swiftllm_hip_paged_attention_v2_workspace_size(
    int num_seqs, int num_heads, int num_kv_heads, int head_dim,
    int block_size, int max_num_blocks_per_seq, int partition_size);

/* Zero-fills `bytes` bytes at `workspace` with a kernel (no memset node, so
 * it may be captured in a graph). No workspace of this library needs it; it
 * is there for callers that want deterministic scratch contents. */
int swiftllm_hip_workspace_clear(void* workspace, size_t bytes,
                                 hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 2. Status-returning twins of the launchers (same arguments; return a     */
/*    swiftllm_status). num_blocks bounds every block id read from           */
/*    block_tables / slot_mapping: ids outside [0, num_blocks) are skipped.  */
/*    Pass num_blocks <= 0 when the pool size is unknown (no bound);         */
/*    negative ids are skipped in either case.                               */
/* ------------------------------------------------------------------------ */
int swiftllm_hip_launch_paged_attention_v1(
    void* output, const void* query, const void* key_cache,
    const void* value_cache, const int* block_tables, const int* context_lens,
    float scale, int num_seqs, int num_heads, int num_kv_heads, int head_dim,
    int block_size, int max_num_blocks_per_seq, int num_blocks,
    hipStream_t stream);

int swiftllm_hip_launch_paged_attention_v2(
    void* output, void* workspace, size_t workspace_bytes, const void* query,
    const void* key_cache, const void* value_cache, const int* block_tables,
    const int* context_lens, float scale, int num_seqs, int num_heads,
    int num_kv_heads, int head_dim, int block_size, int max_num_blocks_per_seq,
    int partition_size, int num_blocks, hipStream_t stream);

int swiftllm_hip_launch_reshape_and_cache(
    const void* key, const void* value, void* key_cache, void* value_cache,
    const int* slot_mapping, int num_tokens, int num_kv_heads, int head_dim,
    int block_size, int num_blocks, hipStream_t stream);

/* Bytes of the static device scratch behind
 * swiftllm_hip_launch_paged_attention_v2_noalloc (one copy per device). The
 * array is part of libswiftllm_hip.so's code object, so every process that
 * runs any kernel of the library on a device holds these 64 MiB there from
 * the code object's load until the process ends, whether or not it ever
 * calls the no-alloc entry point. */
#define SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): swiftllm_hip_launch_paged_attention_v2 without the
 * workspace arguments. Its split-K scratch is a static device array of
 * SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES bytes, reserved on each device when
 * the library's code object loads there (first use of any of its kernels)
 * and held until the process ends; the first call on a device looks up the
 * array's address, and nothing is allocated or freed per call.
 * Sizes whose workspace (swiftllm_hip_paged_attention_v2_workspace_size for
 * the mode the call runs) exceeds that return SWIFTLLM_ERR_INVALID_PARAMETER.
 * All calls on one device share the array: calls that overlap on a device
 * (several streams or host threads) race and must be ordered on one stream. */
int swiftllm_hip_launch_paged_attention_v2_noalloc(
    void* output, const void* query, const void* key_cache,
    const void* value_cache, const int* block_tables, const int* context_lens,
    float scale, int num_seqs, int num_heads, int num_kv_heads, int head_dim,
    int block_size, int max_num_blocks_per_seq, int partition_size,
    int num_blocks, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 3. Params-struct twins of crates/swiftllm-cuda/src/bindings.rs.           */
/*    size_t stands for usize, float for f32.                                */
/* ------------------------------------------------------------------------ */

/* bindings.rs:8-30 (PagedAttentionParams). */
typedef struct swiftllm_paged_attention_params {
    size_t num_seqs;
    size_t num_heads;
    size_t num_kv_heads;
    size_t head_dim;
    size_t block_size;
    float scale;
    size_t max_context_len;
} swiftllm_paged_attention_params;

/* bindings.rs:78-92 (ReshapeCacheParams). */
typedef struct swiftllm_reshape_cache_params {
    size_t num_tokens;
    size_t num_kv_heads;
    size_t head_dim;
    size_t block_size;
} swiftllm_reshape_cache_params;

/* Replaces bindings::paged_attention_decode (bindings.rs:56-76). The row
 * stride of block_tables is ceil(max_context_len / block_size), the only
 * stride the Rust signature can imply. Runs the single-pass kernel. */
int swiftllm_hip_paged_attention_decode(
    void* output, const void* query, const void* key_cache,
    const void* value_cache, const int32_t* block_tables,
    const int32_t* context_lens, const swiftllm_paged_attention_params* params,
    hipStream_t stream);

/* Replaces bindings::reshape_and_cache (bindings.rs:94-113). */
int swiftllm_hip_reshape_and_cache(const void* key, const void* value,
                                   void* key_cache, void* value_cache,
                                   const int32_t* slot_mapping,
                                   const swiftllm_reshape_cache_params* params,
                                   hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 3a. Paged prefill (causal attention over a packed batch of prompts).      */
/* ------------------------------------------------------------------------ */

/* Replaces bindings::paged_attention_prefill (bindings.rs:32-54): the steps
 * of PagedAttention::prefill (paged_attention.rs:154-189) after the K/V
 * write. query / output fp16 [T, H, D] packed: sequence s owns tokens
 * [start_s, start_s + context_lens[s]), start_s the sum of the lengths
 * before it. Token i of s attends to tokens j <= i of s, whose K/V sit in
 * the cache at slot_mapping[start_s + j]; the slots of a sequence must walk
 * its block table from position 0 (table[p / 16] * 16 + p % 16).
 * params->max_context_len bounds every context_lens[s]; above 2^24 tokens it
 * can return SWIFTLLM_ERR_NOT_SUPPORTED (grid size). */
int swiftllm_hip_paged_attention_prefill(
    void* output, const void* query, const void* key_cache,
    const void* value_cache, const int32_t* slot_mapping,
    const int32_t* context_lens, const swiftllm_paged_attention_params* params,
    hipStream_t stream);

/* The same with plain arguments and a pool bound: blocks outside
 * [0, num_blocks) are skipped (num_blocks <= 0: no bound; negative block ids
 * are always skipped). */
int swiftllm_hip_launch_paged_prefill(void* output, const void* query,
                                      const void* key_cache,
                                      const void* value_cache,
                                      const int32_t* slot_mapping,
                                      const int32_t* context_lens, float scale,
                                      int num_seqs, int num_heads,
                                      int num_kv_heads, int head_dim,
                                      int block_size, int max_context_len,
                                      int num_blocks, hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 3b. Block copies of the KV cache. block_mapping holds num_pairs (src, dst) */
/*     int64 pairs in memory the device can read (device memory or pinned    */
/*     host memory). A pair with a negative id is skipped; destinations must */
/*     be distinct and must not be sources in the same call.                 */
/* ------------------------------------------------------------------------ */

/* Replaces launch_copy_blocks (paged_attention.cu:302-327; kernel cu:201-227,
 * whose 2048-thread workgroups fail to launch): K[dst] = K[src] and
 * V[dst] = V[src] for whole [Hkv, D, BS] blocks, one launch. */
void launch_copy_blocks(int64_t* block_mapping, void* key_cache,
                        void* value_cache, int num_pairs, int num_kv_heads,
                        int head_dim, int block_size, hipStream_t stream);

/* Status twin of launch_copy_blocks; ids outside [0, num_blocks) are skipped
 * (num_blocks <= 0: no bound). */
int swiftllm_hip_launch_copy_blocks(const int64_t* block_mapping,
                                    void* key_cache, void* value_cache,
                                    int num_pairs, int num_kv_heads,
                                    int head_dim, int block_size,
                                    int num_blocks, hipStream_t stream);

/* Replaces bindings::copy_blocks (bindings.rs:200-223): the same pairs in
 * the K and V caches of every layer. key_caches / value_caches are host
 * arrays of num_layers device pointers. */
int swiftllm_hip_copy_blocks(void* const* key_caches,
                             void* const* value_caches,
                             const int64_t* block_mapping, size_t num_pairs,
                             size_t num_layers, size_t num_kv_heads,
                             size_t head_dim, size_t block_size,
                             hipStream_t stream);

/* Replaces bindings::swap_blocks (bindings.rs:225-242):
 * dst[dst_id * block_size_bytes, + block_size_bytes) =
 * src[src_id * block_size_bytes, + block_size_bytes) for every pair. src
 * and dst are device memory or pinned host memory (hipHostMalloc), in any
 * combination; one kernel moves every block. */
int swiftllm_hip_swap_blocks(const void* src, void* dst,
                             const int64_t* block_mapping, size_t num_pairs,
                             size_t block_size_bytes, hipStream_t stream);

/* swiftllm_hip_swap_blocks with pool bounds: pairs whose src id is outside
 * [0, src_blocks) or whose dst id is outside [0, dst_blocks) are skipped
 * (a bound <= 0: none). */
int swiftllm_hip_launch_swap_blocks(const void* src, void* dst,
                                    const int64_t* block_mapping,
                                    size_t num_pairs, size_t block_size_bytes,
                                    long long src_blocks, long long dst_blocks,
                                    hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 4. MoE top-k routing and dispatch. The reference has no kernel for this:  */
/*    MoeMlp::forward (crates/swiftllm-models/src/layers/mlp.rs:240-252)     */
/*    names the steps (router logits, top-k, route, combine) and returns     */
/*    zeros. Conventions follow sampling/mod.rs:366-385 (max-subtracted     */
/*    softmax; stable descending order, ties to the lower expert index).    */
/* ------------------------------------------------------------------------ */

/* logits fp32 [T, E] -> expert_ids int32 [T, K] (descending logit, ties to
 * the lower index) and weights fp32 [T, K] = softmax probabilities of the
 * selected experts renormalised to sum to 1. 1 <= K <= E <= 256, K <= 8. */
int swiftllm_hip_moe_route(const float* logits, int num_tokens,
                           int num_experts, int top_k, int32_t* expert_ids,
                           float* weights, hipStream_t stream);

/* Bytes of workspace swiftllm_hip_moe_dispatch needs. */
size_t swiftllm_hip_moe_dispatch_workspace_size(int num_tokens,
                                                int num_experts, int top_k);

/* Expert-contiguous permutation of the routed token copies.
 *   expert_counts[e]      = #{(t,k) : expert_ids[t,k] = e}
 *   expert_offsets[E + 1] = exclusive prefix sum, offsets[E] = T*K
 *   row(t,k)              = offsets[e] + rank of (t,k) among the entries of
 *                           expert e in (t ascending, k ascending) order
 *   x_perm[row(t,k), :]   = x[t, :]          (fp16 bit copy, hidden wide)
 *   inverse[t, k]         = row(t,k)
 *   sorted_token_ids[row] = t
 * `workspace` (swiftllm_hip_moe_dispatch_workspace_size bytes, 256-byte
 * aligned) is plain scratch: no initialisation. Ids outside [0, E) are
 * dropped (inverse = -1). x_perm may be NULL to compute the index arrays
 * only. */
int swiftllm_hip_moe_dispatch(const int32_t* expert_ids, const void* x,
                              int num_tokens, int top_k, int num_experts,
                              int hidden, int32_t* expert_counts,
                              int32_t* expert_offsets, void* x_perm,
                              int32_t* inverse, int32_t* sorted_token_ids,
                              void* workspace, size_t workspace_bytes,
                              hipStream_t stream);

/* swiftllm_hip_moe_route followed by swiftllm_hip_moe_dispatch, with the
 * routing done inside the dispatch's ranking kernel (one launch fewer, and
 * the ids are not re-read). Same outputs as the two calls; the same
 * workspace size. */
int swiftllm_hip_moe_route_dispatch(const float* logits, const void* x,
                                    int num_tokens, int top_k, int num_experts,
                                    int hidden, int32_t* expert_ids,
                                    float* weights, int32_t* expert_counts,
                                    int32_t* expert_offsets, void* x_perm,
                                    int32_t* inverse, int32_t* sorted_token_ids,
                                    void* workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 4b. MoE expert computation: steps 3-4 of MoeMlp::forward                 */
/*     (crates/swiftllm-models/src/layers/mlp.rs:240-246) over GatedMlp      */
/*     experts (mlp.rs:118-160: down(silu(gate(x)) * up(x))), Linear weights  */
/*     [out_features, in_features] (layers/mod.rs:22-24). The reference      */
/*     returns zeros for all of it.                                           */
/* ------------------------------------------------------------------------ */

/* Grouped expert GEMM over expert-contiguous rows: expert e owns rows
 * [expert_offsets[e], expert_offsets[e+1]) of `a` (fp16 [m_total, k], e.g.
 * the dispatch's x_perm) and of `c` (fp16 [m_total, n]).
 *   w2 == NULL: c[rows] = a[rows] . w[e]^T
 *   w2 != NULL: c[rows] = silu(a[rows] . w[e]^T) * (a[rows] . w2[e]^T)
 * w and w2 are fp16 [E, n, k]. fp32 accumulation. Supported (NotSupported
 * otherwise): n % 128 == 0 with w2, n % 256 == 0 without; k % 64 == 0 and
 * k <= 2^21; E <= 256. expert_offsets runs non-decreasing from 0 to m_total
 * (as the dispatch writes it): the grid is sized from m_total. Enqueues up
 * to two kernels on `stream`: whole 256-row tiles, and the experts' tails
 * of at most 128 rows (a decode batch: only the second). */
int swiftllm_hip_moe_expert_gemm(const void* a, const void* w, const void* w2,
                                 const int32_t* expert_offsets,
                                 int num_experts, int m_total, int n, int k,
                                 void* c, hipStream_t stream);

/* out[t, :] = fp16( sum_k weights[t, k] * y[inverse[t, k], :] ), fp32
 * fused multiply-adds in k order; entries with inverse outside
 * [0, y_rows) contribute nothing. y fp16 [y_rows, hidden]; hidden % 8 == 0. */
int swiftllm_hip_moe_combine(const void* y, const float* weights,
                             const int32_t* inverse, int num_tokens, int top_k,
                             int hidden, int y_rows, void* out,
                             hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 5. Block-table gather check: materialise the K and V of (seq, kv_head) as */
/*    contiguous [context_len, head_dim] fp16 arrays through the same tile   */
/*    addressing the decode kernel uses (paged_attention.cu:80-87, 114-116). */
/* ------------------------------------------------------------------------ */
int swiftllm_hip_gather_kv(const void* key_cache, const void* value_cache,
                           const int* block_tables, const int* context_lens,
                           int seq, int kv_head, int num_kv_heads,
                           int head_dim, int block_size,
                           int max_num_blocks_per_seq, int max_context_len,
                           void* k_out, void* v_out, hipStream_t stream);

/* Wave-reduction check: the lane reductions the kernels inline (the
 * reference's 32-lane butterflies, paged_attention.cu:17-31, on 64-lane
 * waves), run on caller data so they can be compared lane by lane with a
 * sequential reference. For each row r < num_rows of x (float [num_rows][64])
 * and xi (int32 [num_rows][64]), lane l writes
 *   out[r][0][l] = max of x[r][l % 16 + 16 k], k = 0..3  (softmax row max)
 *   out[r][1][l] = sum of the same four                  (softmax row sum)
 *   out[r][2][l] = max of x[r][0..63]                    (split-K reduce)
 *   out[r][3][l] = sum of x[r][0..63]
 *   scan[r][l]   = xi[r][0] + ... + xi[r][l]             (dispatch offsets)
 * out is float [num_rows][4][64], scan int32 [num_rows][64]. */
int swiftllm_hip_wave_reduce_check(const float* x, const int32_t* xi,
                                   int num_rows, float* out, int32_t* scan,
                                   hipStream_t stream);

/* ------------------------------------------------------------------------ */
/* 6. Host-side metadata (no device work).                                   */
/* ------------------------------------------------------------------------ */

/* KvCache::get_slot_mapping (crates/swiftllm-core/src/memory/kv_cache.rs:
 * 186-216): out[i] = table[(start + i) / bs] * bs + (start + i) % bs.
 * Returns SWIFTLLM_ERR_INVALID_PARAMETER when a position falls outside the
 * table ("Block ... not allocated") or a slot does not fit in int32. */
int swiftllm_hip_slot_mapping(const uint64_t* block_table, size_t table_len,
                              size_t block_size, size_t start_pos,
                              size_t num_tokens, int32_t* out);

/* Packs per-sequence block tables (Vec<Vec<usize>> in BatchedCacheMetadata,
 * kv_cache.rs:250-286) given in CSR form (table_offsets[num_seqs + 1] into
 * block_ids) into an int32 [num_seqs, max_blocks_per_seq] array padded with
 * 0, and context lengths into int32 [num_seqs]. max_blocks_per_seq must be
 * >= every table length and every ceil(context_len / block_size). */
int swiftllm_hip_pack_block_tables(const uint64_t* block_ids,
                                   const uint64_t* table_offsets,
                                   const uint64_t* context_lens,
                                   size_t num_seqs, size_t block_size,
                                   size_t max_blocks_per_seq,
                                   int32_t* block_tables_out,
                                   int32_t* context_lens_out);

#ifdef __cplusplus
}
#endif

#endif /* SWIFTLLM_HIP_H */
