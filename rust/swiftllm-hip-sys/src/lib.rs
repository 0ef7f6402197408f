//! Raw FFI declarations of `libswiftllm_hip.so`, one for one with
//! `include/swiftllm_hip.h` (a CPU test of this repository parses both and
//! checks that every function, parameter, type and struct field agrees).
//!
//! This crate replaces the `extern` side that `crates/swiftllm-cuda` never
//! had: its `bindings.rs:8-113` declares safe wrappers whose bodies log and
//! return `Ok(())` without calling a kernel. The safe layer over these
//! declarations is the `swiftllm-hip` crate next to this one.
//!
//! Conventions of every entry point (from the header):
//! - pointers are caller-owned device memory on the current HIP device
//!   (pinned host memory where a function says so);
//! - nothing allocates; scratch comes in as a workspace argument;
//! - launches are asynchronous on `stream` (null = the default stream);
//! - arguments are validated on the host before any launch, and a failure
//!   returns one of the `SWIFTLLM_*` status codes below (the `void`
//!   launchers leave it in `swiftllm_hip_last_error()`).

#![no_std]
#![allow(non_camel_case_types)]

use core::ffi::{c_char, c_float, c_int, c_longlong, c_void};

/// `hipStream_t`: an opaque HIP stream handle; null is the default stream.
pub type hipStream_t = *mut c_void;

// Status codes: the CudaError variants of crates/swiftllm-cuda/src/lib.rs:16-42,
// negated, in declaration order.
pub const SWIFTLLM_OK: c_int = 0;
pub const SWIFTLLM_ERR_INIT: c_int = -1;
pub const SWIFTLLM_ERR_KERNEL: c_int = -2;
pub const SWIFTLLM_ERR_MEMORY: c_int = -3;
pub const SWIFTLLM_ERR_INVALID_PARAMETER: c_int = -4;
pub const SWIFTLLM_ERR_DEVICE_NOT_FOUND: c_int = -5;
pub const SWIFTLLM_ERR_NOT_SUPPORTED: c_int = -6;

/// SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES: the static split-K scratch per device.
pub const SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES: usize = 64 << 20;

/// C twin of `PagedAttentionParams` (crates/swiftllm-cuda/src/bindings.rs:8-30).
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct swiftllm_paged_attention_params {
    pub num_seqs: usize,
    pub num_heads: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub block_size: usize,
    pub scale: c_float,
    pub max_context_len: usize,
}

/// C twin of `ReshapeCacheParams` (crates/swiftllm-cuda/src/bindings.rs:78-92).
#[repr(C)]
#[derive(Debug, Clone, Copy)]
pub struct swiftllm_reshape_cache_params {
    pub num_tokens: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub block_size: usize,
}

extern "C" {
    // -- status ---------------------------------------------------------------
    pub fn swiftllm_hip_last_error() -> c_int;
    pub fn swiftllm_hip_last_error_message() -> *const c_char;
    pub fn swiftllm_hip_version() -> *const c_char;
    pub fn swiftllm_hip_device_check() -> c_int;

    // -- drop-in launchers: paged_attention.cu:232-300, hipStream_t for cudaStream_t
    pub fn launch_paged_attention_v1(
        output: *mut c_void, query: *mut c_void, key_cache: *mut c_void,
        value_cache: *mut c_void, block_tables: *mut c_int, context_lens: *mut c_int,
        scale: c_float, num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int,
        head_dim: c_int, block_size: c_int, max_num_blocks_per_seq: c_int,
        stream: hipStream_t,
    );
    pub fn launch_reshape_and_cache(
        key: *mut c_void, value: *mut c_void, key_cache: *mut c_void,
        value_cache: *mut c_void, slot_mapping: *mut c_int, num_tokens: c_int,
        num_kv_heads: c_int, head_dim: c_int, block_size: c_int, stream: hipStream_t,
    );
    /// Split-K decode (the intent of paged_attention_v2_kernel, cu:139-163).
    pub fn launch_paged_attention_v2(
        output: *mut c_void, workspace: *mut c_void, workspace_bytes: usize,
        query: *mut c_void, key_cache: *mut c_void, value_cache: *mut c_void,
        block_tables: *mut c_int, context_lens: *mut c_int, scale: c_float,
        num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int,
        block_size: c_int, max_num_blocks_per_seq: c_int, partition_size: c_int,
        stream: hipStream_t,
    );
    pub fn swiftllm_hip_paged_attention_v2_workspace_size(
        num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int,
        block_size: c_int, max_num_blocks_per_seq: c_int, partition_size: c_int,
    ) -> usize;
    pub fn swiftllm_hip_workspace_clear(
        workspace: *mut c_void, bytes: usize, stream: hipStream_t,
    ) -> c_int;

    // -- status-returning twins with a pool bound (num_blocks <= 0: none) -------
    pub fn swiftllm_hip_launch_paged_attention_v1(
        output: *mut c_void, query: *const c_void, key_cache: *const c_void,
        value_cache: *const c_void, block_tables: *const c_int, context_lens: *const c_int,
        scale: c_float, num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int,
        head_dim: c_int, block_size: c_int, max_num_blocks_per_seq: c_int,
        num_blocks: c_int, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_launch_paged_attention_v2(
        output: *mut c_void, workspace: *mut c_void, workspace_bytes: usize,
        query: *const c_void, key_cache: *const c_void, value_cache: *const c_void,
        block_tables: *const c_int, context_lens: *const c_int, scale: c_float,
        num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int, head_dim: c_int,
        block_size: c_int, max_num_blocks_per_seq: c_int, partition_size: c_int,
        num_blocks: c_int, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_launch_reshape_and_cache(
        key: *const c_void, value: *const c_void, key_cache: *mut c_void,
        value_cache: *mut c_void, slot_mapping: *const c_int, num_tokens: c_int,
        num_kv_heads: c_int, head_dim: c_int, block_size: c_int, num_blocks: c_int,
        stream: hipStream_t,
    ) -> c_int;

    /// No counterpart in the reference: split-K decode for callers that cannot
    /// allocate (graph capture, tight serving loops), with its scratch in a
    /// static device array of SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES per device.
    /// Calls that overlap on one device race on that array.
    pub fn swiftllm_hip_launch_paged_attention_v2_noalloc(
        output: *mut c_void, query: *const c_void, key_cache: *const c_void,
        value_cache: *const c_void, block_tables: *const c_int, context_lens: *const c_int,
        scale: c_float, num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int,
        head_dim: c_int, block_size: c_int, max_num_blocks_per_seq: c_int,
        partition_size: c_int, num_blocks: c_int, stream: hipStream_t,
    ) -> c_int;

    // -- params-struct twins of bindings.rs ------------------------------------
    /// bindings.rs:56-76 (paged_attention_decode).
    pub fn swiftllm_hip_paged_attention_decode(
        output: *mut c_void, query: *const c_void, key_cache: *const c_void,
        value_cache: *const c_void, block_tables: *const i32, context_lens: *const i32,
        params: *const swiftllm_paged_attention_params, stream: hipStream_t,
    ) -> c_int;
    /// bindings.rs:94-113 (reshape_and_cache).
    pub fn swiftllm_hip_reshape_and_cache(
        key: *const c_void, value: *const c_void, key_cache: *mut c_void,
        value_cache: *mut c_void, slot_mapping: *const i32,
        params: *const swiftllm_reshape_cache_params, stream: hipStream_t,
    ) -> c_int;

    // -- paged prefill: bindings.rs:32-54 ----------------------------------------
    pub fn swiftllm_hip_paged_attention_prefill(
        output: *mut c_void, query: *const c_void, key_cache: *const c_void,
        value_cache: *const c_void, slot_mapping: *const i32, context_lens: *const i32,
        params: *const swiftllm_paged_attention_params, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_launch_paged_prefill(
        output: *mut c_void, query: *const c_void, key_cache: *const c_void,
        value_cache: *const c_void, slot_mapping: *const i32, context_lens: *const i32,
        scale: c_float, num_seqs: c_int, num_heads: c_int, num_kv_heads: c_int,
        head_dim: c_int, block_size: c_int, max_context_len: c_int, num_blocks: c_int,
        stream: hipStream_t,
    ) -> c_int;

    // -- block copies: cu:302-327, bindings.rs:200-242 ---------------------------
    pub fn launch_copy_blocks(
        block_mapping: *mut i64, key_cache: *mut c_void, value_cache: *mut c_void,
        num_pairs: c_int, num_kv_heads: c_int, head_dim: c_int, block_size: c_int,
        stream: hipStream_t,
    );
    pub fn swiftllm_hip_launch_copy_blocks(
        block_mapping: *const i64, key_cache: *mut c_void, value_cache: *mut c_void,
        num_pairs: c_int, num_kv_heads: c_int, head_dim: c_int, block_size: c_int,
        num_blocks: c_int, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_copy_blocks(
        key_caches: *const *mut c_void, value_caches: *const *mut c_void,
        block_mapping: *const i64, num_pairs: usize, num_layers: usize,
        num_kv_heads: usize, head_dim: usize, block_size: usize, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_swap_blocks(
        src: *const c_void, dst: *mut c_void, block_mapping: *const i64,
        num_pairs: usize, block_size_bytes: usize, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_launch_swap_blocks(
        src: *const c_void, dst: *mut c_void, block_mapping: *const i64,
        num_pairs: usize, block_size_bytes: usize, src_blocks: c_longlong,
        dst_blocks: c_longlong, stream: hipStream_t,
    ) -> c_int;

    // -- MoE routing site of MoeMlp::forward (mlp.rs:240-252) ---------------------
    pub fn swiftllm_hip_moe_route(
        logits: *const c_float, num_tokens: c_int, num_experts: c_int, top_k: c_int,
        expert_ids: *mut i32, weights: *mut c_float, stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_moe_dispatch_workspace_size(
        num_tokens: c_int, num_experts: c_int, top_k: c_int,
    ) -> usize;
    pub fn swiftllm_hip_moe_dispatch(
        expert_ids: *const i32, x: *const c_void, num_tokens: c_int, top_k: c_int,
        num_experts: c_int, hidden: c_int, expert_counts: *mut i32,
        expert_offsets: *mut i32, x_perm: *mut c_void, inverse: *mut i32,
        sorted_token_ids: *mut i32, workspace: *mut c_void, workspace_bytes: usize,
        stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_moe_route_dispatch(
        logits: *const c_float, x: *const c_void, num_tokens: c_int, top_k: c_int,
        num_experts: c_int, hidden: c_int, expert_ids: *mut i32, weights: *mut c_float,
        expert_counts: *mut i32, expert_offsets: *mut i32, x_perm: *mut c_void,
        inverse: *mut i32, sorted_token_ids: *mut i32, workspace: *mut c_void,
        workspace_bytes: usize, stream: hipStream_t,
    ) -> c_int;

    // -- MoE expert computation: mlp.rs:240-246 steps 3-4 ------------------------
    pub fn swiftllm_hip_moe_expert_gemm(
        a: *const c_void, w: *const c_void, w2: *const c_void, expert_offsets: *const i32,
        num_experts: c_int, m_total: c_int, n: c_int, k: c_int, c: *mut c_void,
        stream: hipStream_t,
    ) -> c_int;
    pub fn swiftllm_hip_moe_combine(
        y: *const c_void, weights: *const c_float, inverse: *const i32, num_tokens: c_int,
        top_k: c_int, hidden: c_int, y_rows: c_int, out: *mut c_void, stream: hipStream_t,
    ) -> c_int;

    // -- block-table gather check (cu:80-87, 114-116) ----------------------------
    pub fn swiftllm_hip_gather_kv(
        key_cache: *const c_void, value_cache: *const c_void, block_tables: *const c_int,
        context_lens: *const c_int, seq: c_int, kv_head: c_int, num_kv_heads: c_int,
        head_dim: c_int, block_size: c_int, max_num_blocks_per_seq: c_int,
        max_context_len: c_int, k_out: *mut c_void, v_out: *mut c_void, stream: hipStream_t,
    ) -> c_int;

    /// The lane reductions of the kernels on caller rows (max / sum over the
    /// four 16-lane groups, over the wave, and the inclusive scan).
    pub fn swiftllm_hip_wave_reduce_check(
        x: *const c_float, xi: *const i32, num_rows: c_int, out: *mut c_float, scan: *mut i32,
        stream: hipStream_t,
    ) -> c_int;

    // -- host metadata: kv_cache.rs:186-216, 250-286 ------------------------------
    pub fn swiftllm_hip_slot_mapping(
        block_table: *const u64, table_len: usize, block_size: usize, start_pos: usize,
        num_tokens: usize, out: *mut i32,
    ) -> c_int;
    pub fn swiftllm_hip_pack_block_tables(
        block_ids: *const u64, table_offsets: *const u64, context_lens: *const u64,
        num_seqs: usize, block_size: usize, max_blocks_per_seq: usize,
        block_tables_out: *mut i32, context_lens_out: *mut i32,
    ) -> c_int;
}
