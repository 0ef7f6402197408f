"""Loader for libswiftllm_ceilings.so (include/swiftllm_ceilings.h): the
measurement kernels bench.py times beside the path's kernels, on the same
inputs, to give each one the ceiling of its own memory access pattern.

These are not part of the drop-in interface; the product path never loads
this library.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

LIB_PATH = Path(os.environ.get("SWIFTLLM_CEILINGS_LIB")
                or Path(__file__).resolve().parent / "libswiftllm_ceilings.so")

vp = ctypes.c_void_p
i32 = ctypes.c_int
sz = ctypes.c_size_t

SIGNATURES = {
    "swiftllm_ceil_read_stream": (i32, [vp, sz, vp, vp]),
    "swiftllm_ceil_tile_gather": (i32, [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, i32, vp, vp]),
    "swiftllm_ceil_cache_store": (i32, [vp, vp, vp, i32, i32, i32, i32, i32, vp]),
    "swiftllm_ceil_row_copy": (i32, [vp, vp, vp, i32, i32, i32, i32, vp]),
    "swiftllm_ceil_mfma_stream": (i32, [vp, sz, i32, i32, vp, vp]),
}

# FLOP of one workgroup-stage of the MFMA stream: 8 waves x 32
# v_mfma_f32_32x32x16_f16 of 2 * 32 * 32 * 16 FLOP.
MFMA_FLOP_PER_GROUP_STAGE = 8 * 32 * 2 * 32 * 32 * 16

# cache_store modes
STORE_4_ROWS_PER_LANE = 0   # each thread: four 2-byte stores to rows d .. d+3
STORE_LINE_PER_4_LANES = 1  # consecutive lanes: consecutive rows, one store each
STORE_WHOLE_ROWS = 2        # every touched 32-byte row written whole

_LIB: Optional[ctypes.CDLL] = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} is missing: build with `python -m swiftllm_amd.build`")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what}: status {rc}")


def read_stream(src, nbytes: int, sink, stream=None) -> None:
    _check(lib().swiftllm_ceil_read_stream(src.ptr, nbytes, sink.ptr, _h(stream)), "read_stream")


def tile_gather(kc, vc, bt, items, num_items: int, num_seqs: int, num_kv_heads: int, head_dim: int,
                max_num_blocks_per_seq: int, num_blocks: int, load_bytes: int, sink,
                stream=None) -> None:
    _check(lib().swiftllm_ceil_tile_gather(kc.ptr, vc.ptr, bt.ptr, items.ptr, num_items, num_seqs,
                                           num_kv_heads, head_dim, max_num_blocks_per_seq,
                                           num_blocks, load_bytes, sink.ptr, _h(stream)),
           "tile_gather")


def cache_store(kc, vc, slots, num_tokens: int, num_kv_heads: int, head_dim: int,
                num_blocks: int, mode: int, stream=None) -> None:
    _check(lib().swiftllm_ceil_cache_store(kc.ptr, vc.ptr, slots.ptr, num_tokens, num_kv_heads,
                                           head_dim, num_blocks, mode, _h(stream)), "cache_store")


def mfma_stream(operands, nbytes: int, num_groups: int, stages: int, sink, stream=None) -> None:
    _check(lib().swiftllm_ceil_mfma_stream(operands.ptr, nbytes, num_groups, stages, sink.ptr,
                                           _h(stream)), "mfma_stream")


def row_copy(src, dst, dst_rows, num_tokens: int, top_k: int, hidden: int, num_dst_rows: int,
             stream=None) -> None:
    _check(lib().swiftllm_ceil_row_copy(src.ptr, dst.ptr, dst_rows.ptr, num_tokens, top_k, hidden,
                                        num_dst_rows, _h(stream)), "row_copy")


def _h(stream):
    return stream.handle if stream is not None else None


def unit_order(context_lens, num_kv_heads: int, cus: int, snake: bool = True):
    """(sequence, kv head) units longest-first, as int32 s * Hkv + h. With
    `snake`, the list is cut into rounds of `cus` units and every other
    round reversed, so that the two units sharing a CU pair a long context
    with a short one (the decode's single-pass order when its grid is
    resident at once)."""
    import numpy as np

    lens = np.asarray(context_lens, np.int64)
    seqs = np.argsort(-lens, kind="stable")
    units = (seqs[:, None] * num_kv_heads + np.arange(num_kv_heads)[None, :]).reshape(-1)
    if snake:
        rounds = [units[i:i + cus] for i in range(0, len(units), cus)]
        units = np.concatenate([r if k % 2 == 0 else r[::-1] for k, r in enumerate(rounds)])
    return units.astype(np.int32)


def gather_items(context_lens, num_kv_heads: int, partition_tokens: int, cus: int):
    """Work items (unit, first block, end block) of a decode, int32 [n, 3]:
    with partition_tokens 0 one item per (sequence, kv head) in
    unit_order's snake order (the single-pass grid); otherwise one item per
    partition of partition_tokens tokens of each (sequence, kv head),
    longest first (the split-K items)."""
    import numpy as np

    lens = np.maximum(np.asarray(context_lens, np.int64), 0)
    nblk = (lens + 15) // 16
    if partition_tokens == 0:
        units = unit_order(lens, num_kv_heads, cus)
        s = units // num_kv_heads
        return np.stack([units, np.zeros_like(units), nblk[s].astype(np.int32)], 1).astype(np.int32)
    pb = partition_tokens // 16
    items = []
    for s_, nb in enumerate(nblk):
        for p0 in range(0, int(nb), pb):
            p1 = min(p0 + pb, int(nb))
            for h in range(num_kv_heads):
                items.append((s_ * num_kv_heads + h, p0, p1))
    items = np.array(items, np.int32).reshape(-1, 3)
    order = np.argsort(-(items[:, 2] - items[:, 1]), kind="stable")
    return items[order]
