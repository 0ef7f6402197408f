"""Writes the committed golden fixtures of this directory.

    python tests/golden/make_golden.py

The reference's own tests hold no values for this path (its decode, cache
write and MoE routing are stubs), so these small cases are the committed pin.
Each expected output comes from a computation independent of oracle/:

- decode_small.npz: torch.nn.functional.scaled_dot_product_attention in
  float64 on K/V gathered token by token from the block tables with the cache
  addressing of paged_attention.cu:80-87, 114-116 ([NB, Hkv, D, 16]); GQA map
  kvh = h // (H / Hkv) (cu:52); scale applied to the dot product (cu:95).
  Cache slots past each context, and unused pool blocks, hold NaN.
- cache_small.npz: per-element loops of paged_attention.cu:184-197,
  K[slot // 16, h, d, slot % 16] = key[t, h, d]; negative slots skipped.
- moe_small.npz: per-token sort by (-logit, expert) (stable descending,
  crates/swiftllm-core/src/sampling/mod.rs:367-377), weights
  exp(x_k - x_0) / sum (mod.rs:380-385 over the selected experts), and the
  expert-major (t, k) enumeration of the dispatch.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
BS = 16


def _gathered(cache, table, L, kvh, D):
    out = np.empty((L, D), np.float64)
    for j in range(L):
        b = int(table[j // BS])
        for d in range(D):
            out[j, d] = float(cache[b, kvh, d, j % BS])
    return out


def decode_case(seed, S, H, Hkv, D, ctx, extra_blocks):
    rng = np.random.default_rng(seed)
    ctx = np.array(ctx, np.int32)
    nb = [(int(c) + BS - 1) // BS for c in ctx]
    NB = sum(nb) + extra_blocks
    MB = max(max(nb), 1) + 1
    perm = rng.permutation(NB)
    bt = np.full((S, MB), -7, np.int32)          # padding past the used entries
    used = np.zeros((NB, BS), bool)
    k = 0
    for s in range(S):
        for j in range(nb[s]):
            bt[s, j] = perm[k]
            k += 1
            for o in range(BS):
                if j * BS + o < ctx[s]:
                    used[perm[k - 1], o] = True
    kc = (rng.standard_normal((NB, Hkv, D, BS)) * 0.7).astype(np.float16)
    vc = (rng.standard_normal((NB, Hkv, D, BS)) * 0.7).astype(np.float16)
    for b in range(NB):
        for o in range(BS):
            if not used[b, o]:
                kc[b, :, :, o] = np.nan
                vc[b, :, :, o] = np.nan
    q = (rng.standard_normal((S, H, D)) * 0.7).astype(np.float16)
    scale = float(np.float32(1.0) / np.sqrt(np.float32(D)))
    out = np.zeros((S, H, D), np.float64)
    G = H // Hkv
    for s in range(S):
        L = int(ctx[s])
        if L == 0:
            continue
        for kvh in range(Hkv):
            K = torch.from_numpy(_gathered(kc, bt[s], L, kvh, D))
            V = torch.from_numpy(_gathered(vc, bt[s], L, kvh, D))
            Q = torch.from_numpy(q[s, kvh * G:(kvh + 1) * G].astype(np.float64))
            o = torch.nn.functional.scaled_dot_product_attention(
                Q[None], K[None], V[None], scale=scale)[0]
            out[s, kvh * G:(kvh + 1) * G] = o.numpy()
    return dict(q=q, key_cache=kc, value_cache=vc, block_tables=bt, context_lens=ctx,
                scale=np.float32(scale), expected=out)


def cache_case(seed, T, Hkv, D, NB):
    rng = np.random.default_rng(seed)
    slots = rng.choice(NB * BS, size=T, replace=False).astype(np.int32)
    slots[::5] = -1
    key = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    value = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    kc0 = rng.standard_normal((NB, Hkv, D, BS)).astype(np.float16)
    vc0 = rng.standard_normal((NB, Hkv, D, BS)).astype(np.float16)
    kc, vc = kc0.copy(), vc0.copy()
    for t in range(T):
        if slots[t] < 0:
            continue
        b, o = int(slots[t]) // BS, int(slots[t]) % BS
        for h in range(Hkv):
            for d in range(D):
                kc[b, h, d, o] = key[t, h, d]
                vc[b, h, d, o] = value[t, h, d]
    return dict(key=key, value=value, slot_mapping=slots, key_cache_in=kc0, value_cache_in=vc0,
                key_cache_expected=kc, value_cache_expected=vc)


def moe_case(seed, T, E, K, hidden):
    rng = np.random.default_rng(seed)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[1] = 0.25                                  # all tied
    logits[2, : E // 2] = logits[2, E - 1]            # partial ties
    x = rng.standard_normal((T, hidden)).astype(np.float16)
    ids = np.zeros((T, K), np.int32)
    w = np.zeros((T, K), np.float64)
    for t in range(T):
        row = [float(v) for v in logits[t]]
        order = sorted(range(E), key=lambda e: (-row[e], e))[:K]
        ex = [math.exp(row[e] - row[order[0]]) for e in order]
        ids[t] = order
        w[t] = [v / sum(ex) for v in ex]
    rows = [(t, k) for e in range(E) for t in range(T) for k in range(K) if ids[t, k] == e]
    counts = np.array([sum(1 for t in range(T) for k in range(K) if ids[t, k] == e)
                       for e in range(E)], np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    inverse = np.zeros((T, K), np.int32)
    for r, (t, k) in enumerate(rows):
        inverse[t, k] = r
    sorted_ids = np.array([t for t, _ in rows], np.int32)
    return dict(logits=logits, x=x, top_k=np.int32(K), expert_ids=ids, weights=w, counts=counts,
                offsets=offsets, inverse=inverse, sorted_token_ids=sorted_ids,
                x_perm=x[sorted_ids])


def main():
    cases = {
        # G = 4, D = 64; contexts around block edges, one empty sequence
        "a": decode_case(11, S=5, H=8, Hkv=2, D=64, ctx=[1, 16, 17, 70, 0], extra_blocks=2),
        # G = 8, D = 128, one kv head
        "b": decode_case(12, S=2, H=8, Hkv=1, D=128, ctx=[33, 5], extra_blocks=1),
    }
    np.savez_compressed(HERE / "decode_small.npz",
                        **{f"{c}_{k}": v for c, d in cases.items() for k, v in d.items()})
    np.savez_compressed(HERE / "cache_small.npz", **cache_case(13, T=23, Hkv=2, D=32, NB=4))
    np.savez_compressed(HERE / "moe_small.npz", **moe_case(14, T=37, E=8, K=2, hidden=24))
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
