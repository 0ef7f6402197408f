"""Loader for libswiftllm_hip.so with the C signatures of
include/swiftllm_hip.h. The library is required: there is no fallback path.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

# SWIFTLLM_HIP_LIB names another build of the library (the host-sanitized one
# of swiftllm_amd/sanitize.py); by default the one next to this file.
LIB_PATH = Path(os.environ.get("SWIFTLLM_HIP_LIB") or Path(__file__).resolve().parent / "libswiftllm_hip.so")

_LIB: Optional[ctypes.CDLL] = None

# SWIFTLLM_HIP_NOALLOC_SCRATCH_BYTES of include/swiftllm_hip.h.
NOALLOC_SCRATCH_BYTES = 64 << 20

vp = ctypes.c_void_p
i32 = ctypes.c_int
sz = ctypes.c_size_t
i64 = ctypes.c_longlong
f32 = ctypes.c_float


class PagedAttentionParams(ctypes.Structure):
    """C twin of PagedAttentionParams (crates/swiftllm-cuda/src/bindings.rs:8-30)."""

    _fields_ = [
        ("num_seqs", sz),
        ("num_heads", sz),
        ("num_kv_heads", sz),
        ("head_dim", sz),
        ("block_size", sz),
        ("scale", f32),
        ("max_context_len", sz),
    ]


class ReshapeCacheParams(ctypes.Structure):
    """C twin of ReshapeCacheParams (crates/swiftllm-cuda/src/bindings.rs:78-92)."""

    _fields_ = [
        ("num_tokens", sz),
        ("num_kv_heads", sz),
        ("head_dim", sz),
        ("block_size", sz),
    ]


# name -> (restype, argtypes); mirrors include/swiftllm_hip.h one to one.
SIGNATURES = {
    "swiftllm_hip_last_error": (i32, []),
    "swiftllm_hip_last_error_message": (ctypes.c_char_p, []),
    "swiftllm_hip_version": (ctypes.c_char_p, []),
    "swiftllm_hip_device_check": (i32, []),
    "launch_paged_attention_v1": (None, [vp, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, vp]),
    "launch_reshape_and_cache": (None, [vp, vp, vp, vp, vp, i32, i32, i32, i32, vp]),
    "launch_paged_attention_v2": (
        None, [vp, vp, sz, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_paged_attention_v2_workspace_size": (sz, [i32, i32, i32, i32, i32, i32, i32]),
    "swiftllm_hip_workspace_clear": (i32, [vp, sz, vp]),
    "swiftllm_hip_launch_paged_attention_v1": (
        i32, [vp, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_launch_paged_attention_v2": (
        i32, [vp, vp, sz, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_launch_reshape_and_cache": (i32, [vp, vp, vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_launch_paged_attention_v2_noalloc": (
        i32, [vp, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_paged_attention_decode": (
        i32, [vp, vp, vp, vp, vp, vp, ctypes.POINTER(PagedAttentionParams), vp]),
    "swiftllm_hip_reshape_and_cache": (
        i32, [vp, vp, vp, vp, vp, ctypes.POINTER(ReshapeCacheParams), vp]),
    "swiftllm_hip_moe_route": (i32, [vp, i32, i32, i32, vp, vp, vp]),
    "swiftllm_hip_moe_dispatch_workspace_size": (sz, [i32, i32, i32]),
    "swiftllm_hip_paged_attention_prefill": (i32, [vp, vp, vp, vp, vp, vp, vp, vp]),
    "swiftllm_hip_launch_paged_prefill": (
        i32, [vp, vp, vp, vp, vp, vp, f32, i32, i32, i32, i32, i32, i32, i32, vp]),
    "launch_copy_blocks": (None, [vp, vp, vp, i32, i32, i32, i32, vp]),
    "swiftllm_hip_launch_copy_blocks": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "swiftllm_hip_copy_blocks": (i32, [vp, vp, vp, sz, sz, sz, sz, sz, vp]),
    "swiftllm_hip_swap_blocks": (i32, [vp, vp, vp, sz, sz, vp]),
    "swiftllm_hip_launch_swap_blocks": (i32, [vp, vp, vp, sz, sz, i64, i64, vp]),
    "swiftllm_hip_moe_dispatch": (
        i32, [vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, sz, vp]),
    "swiftllm_hip_moe_route_dispatch": (
        i32, [vp, vp, i32, i32, i32, i32, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
    "swiftllm_hip_moe_expert_gemm": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "swiftllm_hip_moe_combine": (i32, [vp, vp, vp, i32, i32, i32, i32, vp, vp]),
    "swiftllm_hip_gather_kv": (
        i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp, vp]),
    "swiftllm_hip_wave_reduce_check": (i32, [vp, vp, i32, vp, vp, vp]),
    "swiftllm_hip_slot_mapping": (i32, [vp, sz, sz, sz, sz, vp]),
    "swiftllm_hip_pack_block_tables": (i32, [vp, vp, vp, sz, sz, sz, vp, vp]),
}


class LibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library; raises LibraryMissing when it has not been built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise LibraryMissing(
                f"{LIB_PATH} is missing: build it with `python -m swiftllm_amd.build` "
                "(or __graft_entry__.build())")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def last_error() -> tuple[int, str]:
    L = lib()
    return L.swiftllm_hip_last_error(), L.swiftllm_hip_last_error_message().decode()
