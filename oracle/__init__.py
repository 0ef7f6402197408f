"""CPU oracle for the swiftllm decode hot path.

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker (and, for the fp32 C decode, as
the timed CPU baseline). The product package swiftllm_amd never imports it.

Contents, each citing the reference text it restates (paths relative to the
reference repository; "cu:" = crates/swiftllm-cuda/kernels/paged_attention.cu):

  decode_f64 / decode_f32    C (liboracle.so): cu:35-137 contract, textbook
                             softmax attention, fp64 resp. fp32 accumulation
  decode_numpy               numpy fp64 restatement of the same (small cases)
  prefill_numpy              numpy fp64: causal attention over packed prompts
                             whose K/V sit at slot_mapping (bindings.rs:32-54,
                             paged_attention.rs:154-189)
  reshape_and_cache          C and numpy: cu:167-199
  gather_kv                  numpy: cu:80-87, 114-116 block-table gather
  slot_mapping               kv_cache.rs:186-216 (crates/swiftllm-core/src/memory)
  blocks_needed              block_manager.rs:307-309
  moe_route / moe_dispatch   mlp.rs:240-246 steps with sampling/mod.rs:366-385
                             conventions (max-subtracted softmax, stable
                             descending order)
  moe_route_dispatch_serial  C, one thread: the same route (fp32 softmax) and a
                             serial counting sort with the row copies (the MoE
                             CPU baseline)
  copy_blocks / swap_blocks  numpy: cu:201-227 (launcher cu:302-327) and
                             crates/swiftllm-cuda/src/bindings.rs:200-242
  silu / moe_expert_gemm /   numpy: MoeMlp steps 3-4 (mlp.rs:240-246) over
  moe_combine                GatedMlp (mlp.rs:118-160), silu at mlp.rs:263-265,
                             Linear weights [out, in] (layers/mod.rs:22-24)

Which independent checks pin each function is stated in the tests that use
it (tests/test_oracle_*.py); every function here has at least one.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# SWIFTLLM_ORACLE_LIB names another build (the sanitized one, `make -C oracle
# sanitize`); by default liboracle.so here.
LIB_PATH = Path(os.environ.get("SWIFTLLM_ORACLE_LIB") or HERE / "liboracle.so")

_LIB = None


def build() -> Path:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE), "liboracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp = ctypes.c_void_p
        i = ctypes.c_int
        L.oracle_decode_f64.argtypes = [vp, vp, vp, vp, vp, ctypes.c_double, i, i, i, i, i, i, vp]
        L.oracle_decode_f64.restype = None
        L.oracle_decode_f32.argtypes = [vp, vp, vp, vp, vp, ctypes.c_float, i, i, i, i, i, i, vp]
        L.oracle_decode_f32.restype = None
        L.oracle_reshape_and_cache.argtypes = [vp, vp, vp, vp, vp, i, i, i, i]
        L.oracle_reshape_and_cache.restype = None
        L.oracle_max_threads.restype = i
        L.oracle_moe_route_dispatch_serial.argtypes = [vp, vp, i, i, i, i] + [vp] * 7
        L.oracle_moe_route_dispatch_serial.restype = None
        L.oracle_set_threads.argtypes = [i]
        _LIB = L
    return _LIB


def _u16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a)
    if a.dtype == np.float16:
        return a.view(np.uint16)
    assert a.dtype == np.uint16, a.dtype
    return a


def _i32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def decode_f64(q, kc, vc, bt, ctx, scale) -> np.ndarray:
    """C fp64 textbook decode. q [S,H,D] fp16; caches [NB,Hkv,D,BS] fp16;
    bt int32 [S,MB]; ctx int32 [S]. Returns float64 [S,H,D]."""
    q16, k16, v16 = _u16(q), _u16(kc), _u16(vc)
    bt32, ctx32 = _i32(bt), _i32(ctx)
    S, H, D = q.shape
    Hkv, BS = kc.shape[1], kc.shape[3]
    out = np.empty((S, H, D), dtype=np.float64)
    lib().oracle_decode_f64(q16.ctypes.data, k16.ctypes.data, v16.ctypes.data, bt32.ctypes.data,
                            ctx32.ctypes.data, float(scale), S, H, Hkv, D, BS, bt32.shape[1],
                            out.ctypes.data)
    return out


def decode_f32(q, kc, vc, bt, ctx, scale) -> np.ndarray:
    """C fp32 decode (the CPU baseline). Returns float32 [S,H,D]."""
    q16, k16, v16 = _u16(q), _u16(kc), _u16(vc)
    bt32, ctx32 = _i32(bt), _i32(ctx)
    S, H, D = q.shape
    Hkv, BS = kc.shape[1], kc.shape[3]
    out = np.empty((S, H, D), dtype=np.float32)
    lib().oracle_decode_f32(q16.ctypes.data, k16.ctypes.data, v16.ctypes.data, bt32.ctypes.data,
                            ctx32.ctypes.data, float(scale), S, H, Hkv, D, BS, bt32.shape[1],
                            out.ctypes.data)
    return out


def gather_kv(cache, bt_row, L):
    """Block-table gather (cu:80-87, 114-116): the first L tokens of one
    sequence from a [NB, Hkv, D, BS] cache, as [Hkv, L, D]."""
    BS = cache.shape[3]
    nblk = (L + BS - 1) // BS
    blocks = np.asarray(bt_row[:nblk], dtype=np.int64)
    tiles = cache[blocks]                      # [nblk, Hkv, D, BS]
    seq = tiles.transpose(1, 0, 3, 2)          # [Hkv, nblk, BS, D]
    return seq.reshape(cache.shape[1], nblk * BS, cache.shape[2])[:, :L, :]


def decode_numpy(q, kc, vc, bt, ctx, scale, kv_head_of=None) -> np.ndarray:
    """numpy fp64 decode; kv_head_of(h, H, Hkv) defaults to h // (H // Hkv)
    (cu:52). Returns float64 [S,H,D]."""
    S, H, D = q.shape
    Hkv = kc.shape[1]
    G = H // Hkv
    out = np.zeros((S, H, D), dtype=np.float64)
    for s in range(S):
        L = max(int(ctx[s]), 0)
        if L == 0:
            continue
        K = gather_kv(kc, bt[s], L).astype(np.float64)
        V = gather_kv(vc, bt[s], L).astype(np.float64)
        for h in range(H):
            kvh = kv_head_of(h, H, Hkv) if kv_head_of else h // G
            logit = (K[kvh] @ q[s, h].astype(np.float64)) * scale
            p = np.exp(logit - logit.max())
            out[s, h] = (p @ V[kvh]) / p.sum()
    return out


def prefill_numpy(q, kc, vc, slot_mapping, context_lens, scale) -> np.ndarray:
    """Steps 1-4 of paged_attention.rs:154-189 in float64: sequence s owns
    the packed tokens [start_s, start_s + L_s); token i attends to tokens
    j <= i of its sequence, whose K/V are read at slot_mapping (cache element
    (slot // BS, kvh, d, slot % BS), cu:80-87 addressing); kvh = h // (H / Hkv)."""
    T, H, D = q.shape
    BS = kc.shape[3]
    Hkv = kc.shape[1]
    G = H // Hkv
    out = np.zeros((T, H, D), np.float64)
    start = 0
    for L in np.maximum(np.asarray(context_lens, dtype=np.int64), 0):
        L = int(L)
        if L:
            sl = np.asarray(slot_mapping[start:start + L], dtype=np.int64)
            b, o = sl // BS, sl % BS
            K = kc[b, :, :, o].astype(np.float64)   # [L, Hkv, D]
            V = vc[b, :, :, o].astype(np.float64)
            mask = np.tril(np.ones((L, L), bool))
            for h in range(H):
                qh = q[start:start + L, h].astype(np.float64)
                sc = (qh @ K[:, h // G].T) * scale
                sc = np.where(mask, sc, -np.inf)
                sc -= sc.max(axis=1, keepdims=True)
                p = np.exp(sc)
                p /= p.sum(axis=1, keepdims=True)
                out[start:start + L, h] = p @ V[:, h // G]
        start += L
    return out


def reshape_and_cache(key, value, kc, vc, slot_mapping) -> None:
    """C restatement of cu:167-199, in place on kc / vc (fp16 or uint16)."""
    k16, v16 = _u16(key), _u16(value)
    kcu, vcu = kc.view(np.uint16), vc.view(np.uint16)
    assert kcu.flags.c_contiguous and vcu.flags.c_contiguous
    T, Hkv, D = key.shape
    BS = kc.shape[3]
    sm = _i32(slot_mapping)
    lib().oracle_reshape_and_cache(k16.ctypes.data, v16.ctypes.data, kcu.ctypes.data,
                                   vcu.ctypes.data, sm.ctypes.data, T, Hkv, D, BS)


def reshape_and_cache_numpy(key, value, kc, vc, slot_mapping) -> None:
    """numpy restatement of cu:184-197 (negative slots skipped)."""
    BS = kc.shape[3]
    sm = np.asarray(slot_mapping, dtype=np.int64)
    t = np.nonzero(sm >= 0)[0]
    b, o = sm[t] // BS, sm[t] % BS
    kc[b, :, :, o] = key[t]
    vc[b, :, :, o] = value[t]


def copy_blocks(key_caches, value_caches, block_mapping) -> None:
    """cu:201-227 (and the per-layer form of bindings.rs:200-223), in place:
    for each (src, dst) pair, the whole [Hkv, D, BS] block of every K and V
    cache is copied from src to dst. Pairs with a negative id are skipped."""
    for src, dst in np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2):
        if src < 0 or dst < 0:
            continue
        for c in list(key_caches) + list(value_caches):
            c[dst] = c[src]


def swap_blocks(src, dst, block_mapping, block_size_bytes: int) -> None:
    """bindings.rs:225-242 on byte views, in place: block dst_id of `dst`
    takes the block_size_bytes bytes of block src_id of `src`."""
    s8 = np.asarray(src).reshape(-1).view(np.uint8)
    d8 = dst.reshape(-1).view(np.uint8)
    n = block_size_bytes
    for a, b in np.asarray(block_mapping, dtype=np.int64).reshape(-1, 2):
        if a < 0 or b < 0:
            continue
        d8[b * n:(b + 1) * n] = s8[a * n:(a + 1) * n]


def silu(x):
    """mlp.rs:263-265: x / (1 + exp(-x)), in float64."""
    x = np.asarray(x, dtype=np.float64)
    return x / (1.0 + np.exp(-x))


def moe_expert_gemm(a, w, w2, offsets):
    """For each expert e, rows [offsets[e], offsets[e+1]) of a (fp16
    [m_total, k]) times w[e]^T (Linear layout [n, k]); with w2 the GatedMlp
    product silu(a.w^T) * (a.w2^T). float64 result [m_total, n]."""
    a = np.asarray(a, dtype=np.float64)
    out = np.zeros((a.shape[0], w.shape[1]), np.float64)
    for e in range(w.shape[0]):
        r0, r1 = int(offsets[e]), int(offsets[e + 1])
        if r1 <= r0:
            continue
        g = a[r0:r1] @ np.asarray(w[e], dtype=np.float64).T
        if w2 is not None:
            g = silu(g) * (a[r0:r1] @ np.asarray(w2[e], dtype=np.float64).T)
        out[r0:r1] = g
    return out


def moe_combine(y, weights, inverse):
    """Combine (mlp.rs:245): out[t] = sum_k weights[t, k] * y[inverse[t, k]],
    entries with inverse < 0 skipped. float64 [T, hidden]."""
    y = np.asarray(y, dtype=np.float64)
    inv = np.asarray(inverse)
    w = np.asarray(weights, dtype=np.float64)
    T, K = inv.shape
    out = np.zeros((T, y.shape[1]), np.float64)
    for k in range(K):
        ok = inv[:, k] >= 0
        out[ok] += w[ok, k:k + 1] * y[inv[ok, k]]
    return out


def blocks_needed(num_tokens: int, block_size: int) -> int:
    """block_manager.rs:307-309."""
    return (num_tokens + block_size - 1) // block_size


def slot_mapping(block_table, block_size: int, start_pos: int, num_tokens: int) -> list[int]:
    """kv_cache.rs:186-216; raises KeyError for an unallocated block (:203-208)."""
    out = []
    for pos in range(start_pos, start_pos + num_tokens):
        block_idx, block_offset = divmod(pos, block_size)
        if block_idx >= len(block_table):
            raise KeyError(f"Block {block_idx} not allocated")
        out.append(block_table[block_idx] * block_size + block_offset)
    return out


def moe_route(logits: np.ndarray, top_k: int):
    """Router (mlp.rs:241-243) with sampling conventions: softmax with the max
    subtracted (sampling/mod.rs:380-385), top-k by a stable descending sort
    (:367-377, ties keep the lower index), weights renormalised over the
    selected experts. fp64. Returns (ids int32 [T,K], weights float64 [T,K])."""
    x = np.asarray(logits, dtype=np.float64)
    order = np.argsort(-x, axis=1, kind="stable")[:, :top_k]
    e = np.exp(x - x.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    sel = np.take_along_axis(p, order, axis=1)
    return order.astype(np.int32), sel / sel.sum(axis=1, keepdims=True)


def moe_dispatch(ids: np.ndarray, num_experts: int):
    """Stable counting sort of the (token, k) entries by expert
    (mlp.rs:244 "route tokens to experts"). Entries with an id outside
    [0, E) are dropped (inverse -1). Returns counts [E], offsets [E+1],
    inverse [T,K], sorted_token_ids [#kept]."""
    ids = np.asarray(ids)
    T, K = ids.shape
    flat = ids.reshape(-1)
    keep = (flat >= 0) & (flat < num_experts)
    counts = np.bincount(flat[keep], minlength=num_experts).astype(np.int32)
    offsets = np.zeros(num_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    inverse = np.full(T * K, -1, dtype=np.int32)
    sorted_ids = np.empty(int(offsets[-1]), dtype=np.int32)
    fill = offsets[:-1].copy()
    for idx in range(T * K):          # (t asc, k asc)
        e = flat[idx]
        if 0 <= e < num_experts:
            row = fill[e]
            fill[e] += 1
            inverse[idx] = row
            sorted_ids[row] = idx // K
    return counts, offsets, inverse.reshape(T, K), sorted_ids


def moe_route_dispatch_serial(logits: np.ndarray, x: np.ndarray, top_k: int):
    """C restatement (one thread) of moe_route + moe_dispatch + the row copy:
    fp32 softmax, k argmax passes with ties to the lower index, a serial
    counting sort. Returns (ids, weights fp32, counts, offsets, x_perm,
    inverse, sorted_token_ids)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    xs = _u16(x)
    T, E = lg.shape
    hidden = xs.shape[1]
    ids = np.empty((T, top_k), np.int32)
    w = np.empty((T, top_k), np.float32)
    counts = np.empty(E, np.int32)
    offsets = np.empty(E + 1, np.int32)
    x_perm = np.empty((T * top_k, hidden), np.uint16)
    inverse = np.empty((T, top_k), np.int32)
    sorted_ids = np.empty(T * top_k, np.int32)
    lib().oracle_moe_route_dispatch_serial(lg.ctypes.data, xs.ctypes.data, T, E, top_k, hidden,
                                           ids.ctypes.data, w.ctypes.data, counts.ctypes.data,
                                           offsets.ctypes.data, x_perm.ctypes.data,
                                           inverse.ctypes.data, sorted_ids.ctypes.data)
    return ids, w, counts, offsets, x_perm.view(np.float16), inverse, sorted_ids
