"""Seeded synthetic inputs for the five workloads the path is measured and
checked on (Llama-3 decode shapes, split-K long context, a ragged
continuous-batching step, Mixtral-style MoE dispatch).

All arrays are numpy on the host; callers upload them. Values are drawn with
numpy's PCG64 generator from an explicit seed, so a (config, seed) pair always
yields the same arrays.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import numpy as np

BLOCK_SIZE = 16


@dataclass
class DecodeWorkload:
    name: str
    q: np.ndarray            # fp16 [S, H, D]
    key_cache: np.ndarray    # fp16 [NB, Hkv, D, BS]
    value_cache: np.ndarray  # fp16 [NB, Hkv, D, BS]
    block_tables: np.ndarray  # int32 [S, MB]
    context_lens: np.ndarray  # int32 [S]
    scale: float
    partition_size: int = 512
    # ragged step only: the new token's K/V and its slot
    new_key: Optional[np.ndarray] = None    # fp16 [S, Hkv, D]
    new_value: Optional[np.ndarray] = None
    slot_mapping: Optional[np.ndarray] = None  # int32 [S]

    @property
    def shape(self):
        S, H, D = self.q.shape
        return dict(num_seqs=S, num_heads=H, num_kv_heads=self.key_cache.shape[1], head_dim=D,
                    block_size=self.key_cache.shape[3], max_num_blocks_per_seq=self.block_tables.shape[1],
                    num_blocks=self.key_cache.shape[0])

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes read by one decode: valid tokens only."""
        Hkv, D = self.key_cache.shape[1], self.key_cache.shape[2]
        return int(np.maximum(self.context_lens, 0).astype(np.int64).sum()) * Hkv * D * 2 * 2

    def other_bytes(self) -> int:
        """Q in, O out, block tables, context lengths."""
        S, H, D = self.q.shape
        return 2 * S * H * D * 2 + self.block_tables.nbytes + self.context_lens.nbytes


def _normal_f16(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    out = np.empty(shape, dtype=np.float16)
    flat = out.reshape(-1)
    chunk = 1 << 24
    for i in range(0, flat.size, chunk):
        n = min(chunk, flat.size - i)
        x = rng.standard_normal(n, dtype=np.float32)
        if std != 1.0:
            x *= np.float32(std)
        flat[i:i + n] = x.astype(np.float16)
    return out


def _tables(rng: np.random.Generator, ctx: np.ndarray, num_blocks: int, mb: Optional[int] = None):
    """Block tables drawn from a seeded permutation of the pool, padded with 0."""
    need = (ctx + BLOCK_SIZE - 1) // BLOCK_SIZE
    MB = int(mb if mb is not None else max(int(need.max()), 1))
    perm = rng.permutation(num_blocks).astype(np.int32)
    bt = np.zeros((len(ctx), MB), dtype=np.int32)
    pos = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[pos:pos + n]
        pos += n
    assert pos <= num_blocks
    return bt


def decode_config(cfg: int, seed: int = 0, *, num_seqs: Optional[int] = None,
                  ctx: Optional[int] = None) -> DecodeWorkload:
    """Configs 1-4. num_seqs / ctx override the batch size / a fixed context
    length (for reduced-size tests)."""
    rng = np.random.default_rng(seed)
    if cfg == 1:    # tiny MHA, D64
        S, H, Hkv, D, std = 4, 8, 8, 64, 1.0
        S = num_seqs or S
        lens = rng.integers(1, 257, size=S).astype(np.int32) if ctx is None else np.full(S, ctx, np.int32)
        need = int(((lens + 15) // 16).sum())
        NB = max(128, need)
    elif cfg == 2:  # Llama-3-8B decode
        S, H, Hkv, D, std = 64, 32, 8, 128, 0.5
        S = num_seqs or S
        lens = rng.integers(512, 4097, size=S).astype(np.int32) if ctx is None else np.full(S, ctx, np.int32)
        need = int(((lens + 15) // 16).sum())
        NB = int(math.ceil(1.25 * need))
    elif cfg == 3:  # Llama-3-70B long-context split-K
        S, H, Hkv, D, std = 8, 64, 8, 128, 1.0
        S = num_seqs or S
        lens = np.full(S, 32768 if ctx is None else ctx, np.int32)
        need = int(((lens + 15) // 16).sum())
        NB = need
    elif cfg == 4:  # ragged continuous-batching step
        S, H, Hkv, D, std = 256, 32, 8, 128, 1.0
        S = num_seqs or S
        if ctx is None:
            lens = np.exp(rng.normal(math.log(600.0), 1.0, size=S))
            lens = np.clip(np.rint(lens), 1, 8192).astype(np.int32)
            # at least 1/8 of the sequences open a fresh block with the new token
            opens = rng.choice(S, size=max(1, S // 8), replace=False)
            lens[opens] = np.clip((lens[opens] // 16) * 16 + 1, 1, 8192)
        else:
            lens = np.full(S, ctx, np.int32)
        need = int(((lens + 15) // 16).sum())
        NB = int(math.ceil(1.25 * need))
    else:
        raise ValueError(f"decode config {cfg}")
    bt = _tables(rng, lens, NB)
    kc = _normal_f16(rng, (NB, Hkv, D, BLOCK_SIZE), std)
    vc = _normal_f16(rng, (NB, Hkv, D, BLOCK_SIZE), std)
    q = _normal_f16(rng, (S, H, D), std)
    if cfg == 3:
        # one outlier channel per kv head, scaled x8, to stress softmax stability
        ch = rng.integers(0, D, size=Hkv)
        for h in range(Hkv):
            kc[:, h, ch[h], :] = (kc[:, h, ch[h], :].astype(np.float32) * 8).astype(np.float16)
    wl = DecodeWorkload(name=f"config{cfg}", q=q, key_cache=kc, value_cache=vc, block_tables=bt,
                        context_lens=lens, scale=1.0 / math.sqrt(D))
    if cfg == 4:
        # the new token of each sequence sits at position ctx - 1
        pos = lens - 1
        wl.slot_mapping = (bt[np.arange(S), pos // 16] * 16 + pos % 16).astype(np.int32)
        wl.new_key = _normal_f16(rng, (S, Hkv, D), std)
        wl.new_value = _normal_f16(rng, (S, Hkv, D), std)
    return wl


@dataclass
class PrefillWorkload:
    q: np.ndarray             # fp16 [T, H, D] packed prompts
    key_cache: np.ndarray     # fp16 [NB, Hkv, D, BS], the prompts' K/V already written
    value_cache: np.ndarray
    slot_mapping: np.ndarray  # int32 [T]
    context_lens: np.ndarray  # int32 [S] prompt lengths
    key: np.ndarray           # fp16 [T, Hkv, D] (what was written)
    value: np.ndarray
    scale: float

    @property
    def num_tokens(self) -> int:
        return self.q.shape[0]

    def flops(self) -> int:
        """QK^T and PV multiply-adds of the causal attention."""
        T, H, D = self.q.shape
        pairs = sum(int(L) * (int(L) + 1) // 2 for L in self.context_lens)
        return 4 * pairs * H * D

    def bytes(self) -> int:
        """Q in, O out, K/V read once per sequence and kv head."""
        T, H, D = self.q.shape
        Hkv = self.key_cache.shape[1]
        return 2 * T * H * D * 2 + 2 * T * Hkv * D * 2 + self.slot_mapping.nbytes


def prefill_config(lens, num_heads: int = 32, num_kv_heads: int = 8, head_dim: int = 128,
                   seed: int = 0, std: float = 0.5, poison: bool = True) -> PrefillWorkload:
    """Packed prompts of the given lengths over a randomly permuted block pool
    (1.25x the blocks needed); slots walk each prompt's table from position 0
    (kv_cache.rs:186-216). Unused cache slots hold NaN when `poison`."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    T = int(lens.sum())
    need = int(((lens + BLOCK_SIZE - 1) // BLOCK_SIZE).sum())
    NB = max(int(math.ceil(1.25 * need)), 1)
    perm = rng.permutation(NB)
    slots, k = [], 0
    for L in lens:
        nb = (int(L) + BLOCK_SIZE - 1) // BLOCK_SIZE
        table = perm[k:k + nb]
        k += nb
        slots.extend(int(table[p // BLOCK_SIZE]) * BLOCK_SIZE + p % BLOCK_SIZE for p in range(int(L)))
    slots = np.asarray(slots, dtype=np.int32)
    Hkv, D = num_kv_heads, head_dim
    fill = np.nan if poison else 0.0
    kc = np.full((NB, Hkv, D, BLOCK_SIZE), fill, np.float16)
    vc = np.full((NB, Hkv, D, BLOCK_SIZE), fill, np.float16)
    key = _normal_f16(rng, (T, Hkv, D), std)
    value = _normal_f16(rng, (T, Hkv, D), std)
    b, o = slots // BLOCK_SIZE, slots % BLOCK_SIZE
    kc[b, :, :, o] = key
    vc[b, :, :, o] = value
    q = _normal_f16(rng, (T, num_heads, D), std)
    return PrefillWorkload(q=q, key_cache=kc, value_cache=vc, slot_mapping=slots,
                           context_lens=lens, key=key, value=value, scale=1.0 / math.sqrt(D))


@dataclass
class MoeWorkload:
    x: np.ndarray        # fp16 [T, hidden]
    logits: np.ndarray   # fp32 [T, E]
    top_k: int

    @property
    def num_experts(self) -> int:
        return self.logits.shape[1]

    def bytes(self) -> int:
        T, hidden = self.x.shape
        E, K = self.num_experts, self.top_k
        return 4 * T * E + 2 * T * hidden + 2 * T * K * hidden + T * K * 12 + 4 * (E + 1)


def moe_config(seed: int = 0, *, num_tokens: int = 4096, hidden: int = 4096,
               num_experts: int = 8, top_k: int = 2) -> MoeWorkload:
    """Config 5: Mixtral-8x7B-style dispatch."""
    rng = np.random.default_rng(seed)
    x = _normal_f16(rng, (num_tokens, hidden), 1.0)
    logits = rng.standard_normal((num_tokens, num_experts), dtype=np.float32)
    return MoeWorkload(x=x, logits=logits, top_k=top_k)


def expert_weights(rng: np.random.Generator, num_experts: int, n: int, k: int) -> np.ndarray:
    """fp16 [E, n, k] Linear weights (rows = output features), a different
    matrix for every expert: one N(0, 1/k) matrix whose rows each expert
    takes in its own seeded order. Expert e's output column j is then
    column perm_e[j] of the shared matrix, so a tile computed with another
    expert's weight, or with the right weight at the wrong rows, gives
    different values."""
    base = _normal_f16(rng, (n, k), 1.0 / math.sqrt(k))
    out = np.empty((num_experts, n, k), np.float16)
    for e in range(num_experts):
        np.take(base, rng.permutation(n), axis=0, out=out[e])
    return out
