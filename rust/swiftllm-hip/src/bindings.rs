//! The decode-path functions of crates/swiftllm-cuda/src/bindings.rs with
//! the same names, parameter lists and result type, calling the MI355X
//! kernels of libswiftllm_hip.so where the reference bodies log and return
//! `Ok(())`. The reference signatures carry no stream, so every call goes to
//! the default (null) stream, as they imply.

use crate::{check, Result};
use swiftllm_hip_sys as sys;

/// bindings.rs:8-30.
#[derive(Debug, Clone)]
pub struct PagedAttentionParams {
    pub num_seqs: usize,
    pub num_heads: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub block_size: usize,
    pub scale: f32,
    pub max_context_len: usize,
}

impl PagedAttentionParams {
    fn to_c(&self) -> sys::swiftllm_paged_attention_params {
        sys::swiftllm_paged_attention_params {
            num_seqs: self.num_seqs,
            num_heads: self.num_heads,
            num_kv_heads: self.num_kv_heads,
            head_dim: self.head_dim,
            block_size: self.block_size,
            scale: self.scale,
            max_context_len: self.max_context_len,
        }
    }
}

/// bindings.rs:78-92.
#[derive(Debug, Clone)]
pub struct ReshapeCacheParams {
    pub num_tokens: usize,
    pub num_kv_heads: usize,
    pub head_dim: usize,
    pub block_size: usize,
}

const DEFAULT_STREAM: sys::hipStream_t = std::ptr::null_mut();

/// bindings.rs:32-54. Causal attention over the packed prompts, whose K/V
/// are already in the cache at `slot_mapping`.
pub fn paged_attention_prefill(
    output: *mut half::f16,
    query: *const half::f16,
    key_cache: *const half::f16,
    value_cache: *const half::f16,
    slot_mapping: *const i32,
    context_lens: *const i32,
    params: &PagedAttentionParams,
) -> Result<()> {
    let p = params.to_c();
    check(unsafe {
        sys::swiftllm_hip_paged_attention_prefill(
            output.cast(), query.cast(), key_cache.cast(), value_cache.cast(), slot_mapping,
            context_lens, &p, DEFAULT_STREAM,
        )
    })
}

/// bindings.rs:56-76. Single-pass paged decode; the block-table row stride
/// is ceil(max_context_len / block_size).
pub fn paged_attention_decode(
    output: *mut half::f16,
    query: *const half::f16,
    key_cache: *const half::f16,
    value_cache: *const half::f16,
    block_tables: *const i32,
    context_lens: *const i32,
    params: &PagedAttentionParams,
) -> Result<()> {
    let p = params.to_c();
    check(unsafe {
        sys::swiftllm_hip_paged_attention_decode(
            output.cast(), query.cast(), key_cache.cast(), value_cache.cast(), block_tables,
            context_lens, &p, DEFAULT_STREAM,
        )
    })
}

/// bindings.rs:94-113.
pub fn reshape_and_cache(
    key: *const half::f16,
    value: *const half::f16,
    key_cache: *mut half::f16,
    value_cache: *mut half::f16,
    slot_mapping: *const i32,
    params: &ReshapeCacheParams,
) -> Result<()> {
    let p = sys::swiftllm_reshape_cache_params {
        num_tokens: params.num_tokens,
        num_kv_heads: params.num_kv_heads,
        head_dim: params.head_dim,
        block_size: params.block_size,
    };
    check(unsafe {
        sys::swiftllm_hip_reshape_and_cache(
            key.cast(), value.cast(), key_cache.cast(), value_cache.cast(), slot_mapping, &p,
            DEFAULT_STREAM,
        )
    })
}

/// bindings.rs:200-223. `key_caches` / `value_caches` hold one device
/// pointer per layer; `block_mapping` is int64 (src, dst) pairs in memory
/// the device can read.
pub fn copy_blocks(
    key_caches: &[*mut half::f16],
    value_caches: &[*mut half::f16],
    block_mapping: *const i64,
    num_pairs: usize,
    num_layers: usize,
    num_kv_heads: usize,
    head_dim: usize,
    block_size: usize,
) -> Result<()> {
    if key_caches.len() < num_layers || value_caches.len() < num_layers {
        return Err(crate::CudaError::InvalidParameter(format!(
            "copy_blocks: {num_layers} layers but {} key / {} value caches",
            key_caches.len(),
            value_caches.len()
        )));
    }
    check(unsafe {
        sys::swiftllm_hip_copy_blocks(
            key_caches.as_ptr().cast(), value_caches.as_ptr().cast(), block_mapping, num_pairs,
            num_layers, num_kv_heads, head_dim, block_size, DEFAULT_STREAM,
        )
    })
}

/// bindings.rs:225-242. `src` and `dst` are device memory or pinned host
/// memory (hipHostMalloc) in any combination.
pub fn swap_blocks(
    src: *const half::f16,
    dst: *mut half::f16,
    block_mapping: *const i64,
    num_pairs: usize,
    block_size_bytes: usize,
) -> Result<()> {
    check(unsafe {
        sys::swiftllm_hip_swap_blocks(
            src.cast(), dst.cast(), block_mapping, num_pairs, block_size_bytes, DEFAULT_STREAM,
        )
    })
}

/// The routing site of MoeMlp::forward (crates/swiftllm-models/src/layers/
/// mlp.rs:240-252), which has no binding in the reference: router logits
/// fp32 [T, E] to top-k expert ids and renormalised weights, then the
/// expert-contiguous permutation of the token rows. `workspace` holds
/// `moe_dispatch_workspace_size(T, E, K)` bytes.
#[allow(clippy::too_many_arguments)]
pub fn moe_route_dispatch(
    logits: *const f32,
    x: *const half::f16,
    num_tokens: usize,
    top_k: usize,
    num_experts: usize,
    hidden: usize,
    expert_ids: *mut i32,
    weights: *mut f32,
    expert_counts: *mut i32,
    expert_offsets: *mut i32,
    x_perm: *mut half::f16,
    inverse: *mut i32,
    sorted_token_ids: *mut i32,
    workspace: *mut u8,
    workspace_bytes: usize,
) -> Result<()> {
    let n = |v: usize, what: &str| {
        i32::try_from(v)
            .map_err(|_| crate::CudaError::InvalidParameter(format!("{what} does not fit in i32")))
    };
    check(unsafe {
        sys::swiftllm_hip_moe_route_dispatch(
            logits, x.cast(), n(num_tokens, "num_tokens")?, n(top_k, "top_k")?,
            n(num_experts, "num_experts")?, n(hidden, "hidden")?, expert_ids, weights,
            expert_counts, expert_offsets, x_perm.cast(), inverse, sorted_token_ids,
            workspace.cast(), workspace_bytes, DEFAULT_STREAM,
        )
    })
}

/// Bytes of workspace `moe_route_dispatch` needs.
pub fn moe_dispatch_workspace_size(num_tokens: usize, num_experts: usize, top_k: usize) -> usize {
    match (i32::try_from(num_tokens), i32::try_from(num_experts), i32::try_from(top_k)) {
        (Ok(t), Ok(e), Ok(k)) => unsafe { sys::swiftllm_hip_moe_dispatch_workspace_size(t, e, k) },
        _ => usize::MAX,
    }
}
