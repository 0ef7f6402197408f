"""Host-side interface of the decode hot path, mirroring the reference's names.

Reference (paths relative to the swiftllm repository):
  crates/swiftllm-cuda/src/lib.rs:16-42          CudaError variants
  crates/swiftllm-cuda/src/bindings.rs:8-242     PagedAttentionParams,
                                                 paged_attention_decode,
                                                 ReshapeCacheParams,
                                                 reshape_and_cache,
                                                 copy_blocks, swap_blocks
  crates/swiftllm-core/src/memory/paged_attention.rs:18-266
                                                 PagedAttentionConfig,
                                                 PagedAttention
  crates/swiftllm-core/src/memory/kv_cache.rs:14-298
                                                 KvCacheConfig,
                                                 get_slot_mapping,
                                                 BatchedCacheMetadata

Device tensors are swiftllm_amd._hip.DeviceArray (or raw device pointers as
ints); every call goes through libswiftllm_hip.so. There is no CPU path.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass, field
from typing import Optional, Sequence, Union

import numpy as np

from . import _lib
from ._hip import DeviceArray, HostArray, Stream

Ptr = Union[int, DeviceArray, HostArray, None]


# ---------------------------------------------------------------------------
# Errors: lib.rs:16-42. The status value of each is the C ABI's code.
# ---------------------------------------------------------------------------
class CudaError(RuntimeError):
    code = -2

    def __init__(self, message: str = ""):
        super().__init__(message)
        self.message = message


class InitError(CudaError):
    code = -1


class KernelError(CudaError):
    code = -2


class DeviceMemoryError(CudaError):
    """CudaError::MemoryError."""
    code = -3


class InvalidParameter(CudaError):
    code = -4


class DeviceNotFound(CudaError):
    code = -5


class NotSupported(CudaError):
    code = -6


_BY_CODE = {c.code: c for c in (InitError, KernelError, DeviceMemoryError, InvalidParameter,
                                DeviceNotFound, NotSupported)}


def check_status(status: int) -> None:
    """Raises the CudaError subclass for a non-zero status of the C ABI."""
    if status == 0:
        return
    _, msg = _lib.last_error()
    raise _BY_CODE.get(status, CudaError)(msg)


def _p(x: Ptr) -> Optional[int]:
    if x is None:
        return None
    if isinstance(x, (DeviceArray, HostArray)):
        return x.ptr
    return int(x)


def _s(stream: Optional[Stream]) -> Optional[int]:
    return stream.handle if stream is not None else None


# ---------------------------------------------------------------------------
# bindings.rs
# ---------------------------------------------------------------------------
@dataclass
class PagedAttentionParams:
    """bindings.rs:8-30."""
    num_seqs: int
    num_heads: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    scale: float
    max_context_len: int

    def to_c(self) -> _lib.PagedAttentionParams:
        return _lib.PagedAttentionParams(self.num_seqs, self.num_heads, self.num_kv_heads,
                                         self.head_dim, self.block_size, self.scale,
                                         self.max_context_len)


@dataclass
class ReshapeCacheParams:
    """bindings.rs:78-92."""
    num_tokens: int
    num_kv_heads: int
    head_dim: int
    block_size: int

    def to_c(self) -> _lib.ReshapeCacheParams:
        return _lib.ReshapeCacheParams(self.num_tokens, self.num_kv_heads, self.head_dim,
                                       self.block_size)


def paged_attention_decode(output: Ptr, query: Ptr, key_cache: Ptr, value_cache: Ptr,
                           block_tables: Ptr, context_lens: Ptr, params: PagedAttentionParams,
                           stream: Optional[Stream] = None) -> None:
    """bindings.rs:56-76. block_tables row stride = ceil(max_context_len / block_size)."""
    c = params.to_c()
    check_status(_lib.lib().swiftllm_hip_paged_attention_decode(
        _p(output), _p(query), _p(key_cache), _p(value_cache), _p(block_tables),
        _p(context_lens), ctypes.byref(c), _s(stream)))


def paged_attention_prefill(output: Ptr, query: Ptr, key_cache: Ptr, value_cache: Ptr,
                            slot_mapping: Ptr, context_lens: Ptr, params: PagedAttentionParams,
                            stream: Optional[Stream] = None) -> None:
    """bindings.rs:32-54: causal attention over packed prompts whose K/V are
    already in the cache at slot_mapping."""
    c = params.to_c()
    check_status(_lib.lib().swiftllm_hip_paged_attention_prefill(
        _p(output), _p(query), _p(key_cache), _p(value_cache), _p(slot_mapping),
        _p(context_lens), ctypes.byref(c), _s(stream)))


def reshape_and_cache(key: Ptr, value: Ptr, key_cache: Ptr, value_cache: Ptr, slot_mapping: Ptr,
                      params: ReshapeCacheParams, stream: Optional[Stream] = None) -> None:
    """bindings.rs:94-113."""
    c = params.to_c()
    check_status(_lib.lib().swiftllm_hip_reshape_and_cache(
        _p(key), _p(value), _p(key_cache), _p(value_cache), _p(slot_mapping), ctypes.byref(c),
        _s(stream)))


def copy_blocks(key_caches: Sequence[Ptr], value_caches: Sequence[Ptr], block_mapping: Ptr,
                num_pairs: int, num_kv_heads: int, head_dim: int, block_size: int,
                stream: Optional[Stream] = None) -> None:
    """bindings.rs:200-223: the (src, dst) int64 pairs of block_mapping in the
    K and V caches of every layer (one device pointer per layer)."""
    n = len(key_caches)
    if len(value_caches) != n:
        raise InvalidParameter(f"{n} key caches but {len(value_caches)} value caches")
    kc = (ctypes.c_void_p * max(n, 1))(*[_p(k) for k in key_caches])
    vc = (ctypes.c_void_p * max(n, 1))(*[_p(v) for v in value_caches])
    check_status(_lib.lib().swiftllm_hip_copy_blocks(
        ctypes.cast(kc, ctypes.c_void_p), ctypes.cast(vc, ctypes.c_void_p), _p(block_mapping),
        num_pairs, n, num_kv_heads, head_dim, block_size, _s(stream)))


def swap_blocks(src: Ptr, dst: Ptr, block_mapping: Ptr, num_pairs: int, block_size_bytes: int,
                stream: Optional[Stream] = None) -> None:
    """bindings.rs:225-242: block copies between device memory and pinned host
    memory (either side may be either)."""
    check_status(_lib.lib().swiftllm_hip_swap_blocks(
        _p(src), _p(dst), _p(block_mapping), num_pairs, block_size_bytes, _s(stream)))


# ---------------------------------------------------------------------------
# Launcher-level calls (paged_attention.cu:230-327 names plus the split-K and
# MoE extensions), status-checked.
# ---------------------------------------------------------------------------
def launch_copy_blocks(block_mapping: Ptr, key_cache: Ptr, value_cache: Ptr, num_pairs: int,
                       num_kv_heads: int, head_dim: int, block_size: int, num_blocks: int = 0,
                       stream: Optional[Stream] = None) -> None:
    """launch_copy_blocks (paged_attention.cu:302-327) with a pool bound."""
    check_status(_lib.lib().swiftllm_hip_launch_copy_blocks(
        _p(block_mapping), _p(key_cache), _p(value_cache), num_pairs, num_kv_heads, head_dim,
        block_size, num_blocks, _s(stream)))


def launch_swap_blocks(src: Ptr, dst: Ptr, block_mapping: Ptr, num_pairs: int,
                       block_size_bytes: int, src_blocks: int = 0, dst_blocks: int = 0,
                       stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_launch_swap_blocks(
        _p(src), _p(dst), _p(block_mapping), num_pairs, block_size_bytes, src_blocks,
        dst_blocks, _s(stream)))


def paged_attention_v1(output: Ptr, query: Ptr, key_cache: Ptr, value_cache: Ptr,
                       block_tables: Ptr, context_lens: Ptr, scale: float, num_seqs: int,
                       num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                       max_num_blocks_per_seq: int, num_blocks: int = 0,
                       stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_launch_paged_attention_v1(
        _p(output), _p(query), _p(key_cache), _p(value_cache), _p(block_tables),
        _p(context_lens), scale, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
        max_num_blocks_per_seq, num_blocks, _s(stream)))


def paged_attention_v2_workspace_size(num_seqs: int, num_heads: int, num_kv_heads: int,
                                      head_dim: int, block_size: int,
                                      max_num_blocks_per_seq: int, partition_size: int) -> int:
    n = _lib.lib().swiftllm_hip_paged_attention_v2_workspace_size(
        num_seqs, num_heads, num_kv_heads, head_dim, block_size, max_num_blocks_per_seq,
        partition_size)
    if n == 0 and num_seqs > 0:
        check_status(_lib.lib().swiftllm_hip_last_error() or InvalidParameter.code)
    return int(n)


def workspace(nbytes: int, stream: Optional[Stream] = None) -> DeviceArray:
    """A zero-filled device workspace of nbytes bytes (256-byte aligned)."""
    ws = DeviceArray((max(nbytes, 4) + 3) // 4, np.uint32)
    check_status(_lib.lib().swiftllm_hip_workspace_clear(ws.ptr, ws.nbytes, _s(stream)))
    return ws


def paged_attention_v2(output: Ptr, ws: DeviceArray, query: Ptr, key_cache: Ptr,
                       value_cache: Ptr, block_tables: Ptr, context_lens: Ptr, scale: float,
                       num_seqs: int, num_heads: int, num_kv_heads: int, head_dim: int,
                       block_size: int, max_num_blocks_per_seq: int, partition_size: int,
                       num_blocks: int = 0, stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_launch_paged_attention_v2(
        _p(output), ws.ptr, ws.nbytes, _p(query), _p(key_cache), _p(value_cache),
        _p(block_tables), _p(context_lens), scale, num_seqs, num_heads, num_kv_heads, head_dim,
        block_size, max_num_blocks_per_seq, partition_size, num_blocks, _s(stream)))


def launch_paged_prefill(output: Ptr, query: Ptr, key_cache: Ptr, value_cache: Ptr,
                         slot_mapping: Ptr, context_lens: Ptr, scale: float, num_seqs: int,
                         num_heads: int, num_kv_heads: int, head_dim: int, block_size: int,
                         max_context_len: int, num_blocks: int = 0,
                         stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_launch_paged_prefill(
        _p(output), _p(query), _p(key_cache), _p(value_cache), _p(slot_mapping),
        _p(context_lens), scale, num_seqs, num_heads, num_kv_heads, head_dim, block_size,
        max_context_len, num_blocks, _s(stream)))


def launch_reshape_and_cache(key: Ptr, value: Ptr, key_cache: Ptr, value_cache: Ptr,
                             slot_mapping: Ptr, num_tokens: int, num_kv_heads: int,
                             head_dim: int, block_size: int, num_blocks: int = 0,
                             stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_launch_reshape_and_cache(
        _p(key), _p(value), _p(key_cache), _p(value_cache), _p(slot_mapping), num_tokens,
        num_kv_heads, head_dim, block_size, num_blocks, _s(stream)))


def gather_kv(key_cache: Ptr, value_cache: Ptr, block_tables: Ptr, context_lens: Ptr, seq: int,
              kv_head: int, num_kv_heads: int, head_dim: int, block_size: int,
              max_num_blocks_per_seq: int, max_context_len: int, k_out: Ptr, v_out: Ptr,
              stream: Optional[Stream] = None) -> None:
    check_status(_lib.lib().swiftllm_hip_gather_kv(
        _p(key_cache), _p(value_cache), _p(block_tables), _p(context_lens), seq, kv_head,
        num_kv_heads, head_dim, block_size, max_num_blocks_per_seq, max_context_len, _p(k_out),
        _p(v_out), _s(stream)))


# ---------------------------------------------------------------------------
# paged_attention.rs
# ---------------------------------------------------------------------------
@dataclass
class PagedAttentionConfig:
    """paged_attention.rs:18-83."""
    num_heads: int
    num_kv_heads: int
    head_dim: int
    scale: float
    block_size: int
    dtype: str = "float16"
    sliding_window: Optional[int] = None
    use_alibi: bool = False

    @classmethod
    def new(cls, num_heads: int, num_kv_heads: int, head_dim: int,
            block_size: int) -> "PagedAttentionConfig":
        """Default scale 1/sqrt(head_dim) (:53)."""
        scale = float(np.float32(1.0) / np.sqrt(np.float32(head_dim)))
        return cls(num_heads, num_kv_heads, head_dim, scale, block_size)

    def with_scale(self, scale: float) -> "PagedAttentionConfig":
        self.scale = scale
        return self

    def with_sliding_window(self, window: int) -> "PagedAttentionConfig":
        self.sliding_window = window
        return self

    def with_alibi(self) -> "PagedAttentionConfig":
        self.use_alibi = True
        return self

    def num_query_groups(self) -> int:
        """:80-82."""
        return self.num_heads // self.num_kv_heads


class PagedAttention:
    """paged_attention.rs:85-266 on the GPU. decode() first stores the new
    K/V through slot_mapping, then attends over the updated cache (the steps
    listed at paged_attention.rs:229-233). Split-K partitions of
    `partition_size` tokens; the workspace is owned by this object."""

    def __init__(self, config: PagedAttentionConfig, partition_size: int = 512):
        self.config = config
        self.partition_size = partition_size
        self._ws: Optional[DeviceArray] = None

    def _validate(self) -> None:
        c = self.config
        if c.use_alibi or c.sliding_window is not None:
            raise NotSupported("alibi / sliding window are declared by the reference "
                               "(paged_attention.rs:39-43) but implemented by no kernel")
        if c.dtype != "float16":
            raise NotSupported(f"dtype {c.dtype}")

    def _workspace(self, S: int, MB: int, stream) -> DeviceArray:
        c = self.config
        need = paged_attention_v2_workspace_size(S, c.num_heads, c.num_kv_heads, c.head_dim,
                                                 c.block_size, MB, self.partition_size)
        if self._ws is None or self._ws.nbytes < need:
            self._ws = workspace(need, stream)
        return self._ws

    def reshape_and_cache(self, key: DeviceArray, value: DeviceArray, key_cache: DeviceArray,
                          value_cache: DeviceArray, slot_mapping: Sequence[int],
                          stream: Optional[Stream] = None) -> None:
        """paged_attention.rs:243-265 (including the length check :255-262)."""
        num_tokens = int(np.prod(key.shape[:-2]))
        if len(slot_mapping) != num_tokens:
            raise InvalidParameter(f"Slot mapping length {len(slot_mapping)} doesn't match "
                                   f"number of tokens {num_tokens}")
        sm = DeviceArray.from_numpy(np.asarray(slot_mapping, dtype=np.int32))
        c = self.config
        launch_reshape_and_cache(key, value, key_cache, value_cache, sm, num_tokens,
                                 c.num_kv_heads, c.head_dim, c.block_size,
                                 num_blocks=key_cache.shape[0], stream=stream)
        if stream is not None:
            stream.synchronize()

    def prefill(self, query: DeviceArray, key: DeviceArray, value: DeviceArray,
                key_cache: DeviceArray, value_cache: DeviceArray, slot_mapping: Sequence[int],
                stream: Optional[Stream] = None) -> DeviceArray:
        """paged_attention.rs:154-189. query [B,S,H,D], key/value [B,S,Hkv,D]
        fp16 on the device, slot_mapping of the B*S tokens; stores K/V (step 5)
        and returns the causal attention output [B,S,H,D] (steps 1-4)."""
        self._validate()
        if len(query.shape) != 4 or len(key.shape) != 4:
            raise InvalidParameter(f"query and key must be 4-d, got {len(query.shape)}-d "
                                   f"and {len(key.shape)}-d")
        B, S, H, D = query.shape
        c = self.config
        if H != c.num_heads or D != c.head_dim:
            raise InvalidParameter(f"query [.., {H}, {D}] vs config heads {c.num_heads} dim {c.head_dim}")
        self.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, stream)
        out = DeviceArray((B, S, H, D), np.float16)
        sm = DeviceArray.from_numpy(np.asarray(slot_mapping, dtype=np.int32))
        ctx = DeviceArray.from_numpy(np.full(B, S, dtype=np.int32))
        launch_paged_prefill(out, query, key_cache, value_cache, sm, ctx, c.scale, B, H,
                             c.num_kv_heads, D, c.block_size, S, num_blocks=key_cache.shape[0],
                             stream=stream)
        if stream is not None:
            stream.synchronize()
        else:
            from ._hip import synchronize
            synchronize()
        return out

    def decode(self, query: DeviceArray, key: DeviceArray, value: DeviceArray,
               key_cache: DeviceArray, value_cache: DeviceArray,
               block_tables: Sequence[Sequence[int]], context_lens: Sequence[int],
               slot_mapping: Sequence[int], stream: Optional[Stream] = None) -> DeviceArray:
        """paged_attention.rs:205-238. query [B,1,H,D], key/value [B,1,Hkv,D]
        fp16 on the device; returns the output [B,1,H,D]."""
        self._validate()
        if len(query.shape) != 4:
            raise InvalidParameter(f"query must be 4-d, got {len(query.shape)}-d")
        B, _, H, D = query.shape
        c = self.config
        if H != c.num_heads or D != c.head_dim:
            raise InvalidParameter(f"query [.., {H}, {D}] vs config heads {c.num_heads} dim {c.head_dim}")
        meta = BatchedCacheMetadata()
        for table, ctx in zip(block_tables, context_lens):
            meta.add_sequence(SequenceCacheMetadata(cache_len=int(ctx), block_table=list(table)), [])
        bt, ctx = meta.pack(c.block_size)
        self.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, stream)
        out = DeviceArray((B, 1, H, D), np.float16)
        bt_d = DeviceArray.from_numpy(bt)
        ctx_d = DeviceArray.from_numpy(ctx)
        ws = self._workspace(B, bt.shape[1], stream)
        paged_attention_v2(out, ws, query, key_cache, value_cache, bt_d, ctx_d, c.scale, B, H,
                           c.num_kv_heads, D, c.block_size, bt.shape[1], self.partition_size,
                           num_blocks=key_cache.shape[0], stream=stream)
        if stream is not None:
            stream.synchronize()
        else:
            from ._hip import synchronize
            synchronize()
        return out


# ---------------------------------------------------------------------------
# kv_cache.rs / block_manager.rs
# ---------------------------------------------------------------------------
_DTYPE_BYTES = {"float32": 4, "float16": 2, "bfloat16": 2, "float8_e4m3": 1, "float8_e5m2": 1,
                "int8": 1, "int4": 1}   # config.rs:154-181


@dataclass
class KvCacheConfig:
    """kv_cache.rs:14-54."""
    num_layers: int
    num_kv_heads: int
    head_dim: int
    block_size: int
    dtype: str = "float16"

    def block_size_bytes(self) -> int:
        return 2 * self.block_size * self.num_kv_heads * self.head_dim * _DTYPE_BYTES[self.dtype]

    def token_size_bytes(self) -> int:
        return 2 * self.num_kv_heads * self.head_dim * _DTYPE_BYTES[self.dtype]

    def total_size_bytes(self, num_tokens: int) -> int:
        return self.num_layers * num_tokens * self.token_size_bytes()


def blocks_needed(num_tokens: int, block_size: int) -> int:
    """block_manager.rs:307-309."""
    return (num_tokens + block_size - 1) // block_size


def get_slot_mapping(block_table: Sequence[int], block_size: int, start_pos: int,
                     num_tokens: int) -> np.ndarray:
    """kv_cache.rs:186-216 through the library's host routine; int32 slots."""
    table = np.ascontiguousarray(block_table, dtype=np.uint64)
    out = np.empty(max(num_tokens, 1), dtype=np.int32)
    check_status(_lib.lib().swiftllm_hip_slot_mapping(
        table.ctypes.data if table.size else None, table.size, block_size, start_pos, num_tokens,
        out.ctypes.data))
    return out[:num_tokens]


@dataclass
class SequenceCacheMetadata:
    """kv_cache.rs:219-246."""
    cache_len: int = 0
    block_table: list = field(default_factory=list)

    def num_blocks(self) -> int:
        return len(self.block_table)


class BatchedCacheMetadata:
    """kv_cache.rs:248-298, plus pack(): the flattening into the int32
    arrays the kernels read."""

    def __init__(self):
        self.sequences: list[SequenceCacheMetadata] = []
        self.slot_mapping: list[int] = []
        self.context_lens: list[int] = []
        self.max_context_len = 0
        self.block_tables: list[list[int]] = []

    def add_sequence(self, metadata: SequenceCacheMetadata, slot_mapping: Sequence[int]) -> None:
        self.context_lens.append(metadata.cache_len)
        self.max_context_len = max(self.max_context_len, metadata.cache_len)
        self.block_tables.append(list(metadata.block_table))
        self.slot_mapping.extend(slot_mapping)
        self.sequences.append(metadata)

    def batch_size(self) -> int:
        return len(self.sequences)

    def pack(self, block_size: int, max_blocks_per_seq: Optional[int] = None):
        """(block_tables int32 [S, MB], context_lens int32 [S]); MB defaults to
        the longest table / ceil(max_context_len / block_size)."""
        S = len(self.sequences)
        lens = np.asarray(self.context_lens, dtype=np.uint64)
        if max_blocks_per_seq is None:
            longest = max((len(t) for t in self.block_tables), default=0)
            max_blocks_per_seq = max(longest, blocks_needed(self.max_context_len, block_size), 1)
        offsets = np.zeros(S + 1, dtype=np.uint64)
        offsets[1:] = np.cumsum([len(t) for t in self.block_tables], dtype=np.uint64)
        ids = np.ascontiguousarray(
            np.concatenate([np.asarray(t, dtype=np.uint64) for t in self.block_tables])
            if S and offsets[-1] else np.zeros(1, dtype=np.uint64))
        bt = np.zeros((max(S, 1), max_blocks_per_seq), dtype=np.int32)
        ctx = np.zeros(max(S, 1), dtype=np.int32)
        check_status(_lib.lib().swiftllm_hip_pack_block_tables(
            ids.ctypes.data, offsets.ctypes.data, lens.ctypes.data if S else None, S, block_size,
            max_blocks_per_seq, bt.ctypes.data, ctx.ctypes.data))
        return bt[:S], ctx[:S]


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)
