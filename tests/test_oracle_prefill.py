"""Pins for oracle.prefill_numpy (causal attention over packed prompts read
through slot_mapping; bindings.rs:32-54, paged_attention.rs:154-189):
torch's scaled_dot_product_attention(is_causal=True) in float64 on K/V
gathered token by token with separately written cache addressing; closed
forms; the causal invariant; planted mistakes (no causal mask, GQA map
h % Hkv)."""

import numpy as np
import pytest
import torch

import oracle
from swiftllm_amd import workloads


def _gather(cache, slot, kvh):
    return cache[slot // 16, kvh, :, slot % 16].astype(np.float64)


@pytest.mark.parametrize("lens,H,Hkv,D", [((5, 17, 33), 8, 2, 64), ((40,), 4, 4, 32),
                                          ((1, 16, 3), 16, 2, 16)])
def test_prefill_matches_torch_causal_sdpa(lens, H, Hkv, D):
    w = workloads.prefill_config(lens, H, Hkv, D, seed=sum(lens))
    got = oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens,
                               w.scale)
    G, start = H // Hkv, 0
    for L in w.context_lens:
        for h in range(H):
            sl = w.slot_mapping[start:start + L]
            K = np.stack([_gather(w.key_cache, int(x), h // G) for x in sl])
            V = np.stack([_gather(w.value_cache, int(x), h // G) for x in sl])
            Q = w.q[start:start + L, h].astype(np.float64)
            ref = torch.nn.functional.scaled_dot_product_attention(
                torch.from_numpy(Q)[None], torch.from_numpy(K)[None], torch.from_numpy(V)[None],
                is_causal=True, scale=w.scale)[0].numpy()
            assert np.abs(got[start:start + L, h] - ref).max() < 1e-10
        start += L


def test_first_token_sees_only_itself():
    w = workloads.prefill_config((9, 23), 4, 2, 32, seed=3)
    got = oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens,
                               w.scale)
    start = 0
    for L in w.context_lens:
        for h in range(4):
            assert np.allclose(got[start, h], w.value[start, h // 2].astype(np.float64), atol=1e-12)
        start += L


def test_causal_invariant_and_planted_full_attention():
    """Changing token j's K/V leaves every earlier output of its prompt
    unchanged and moves token j's; attention without the mask would move
    the earlier ones."""
    w = workloads.prefill_config((30,), 4, 1, 32, seed=4)
    base = oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens,
                                w.scale)
    j = 17
    kc, vc = w.key_cache.copy(), w.value_cache.copy()
    s = int(w.slot_mapping[j])
    kc[s // 16, :, :, s % 16] += np.float16(1.0)
    vc[s // 16, :, :, s % 16] -= np.float16(2.0)
    moved = oracle.prefill_numpy(w.q, kc, vc, w.slot_mapping, w.context_lens, w.scale)
    assert np.array_equal(moved[:j], base[:j])
    assert not np.allclose(moved[j], base[j])
    # planted: the same prompt without a causal mask changes token 0's output
    L = 30
    K = w.key.astype(np.float64)[:, 0]
    V = w.value.astype(np.float64)[:, 0]
    sc = w.q[0, 0].astype(np.float64) @ K.T * w.scale
    p = np.exp(sc - sc.max())
    full = (p / p.sum()) @ V
    assert not np.allclose(full, base[0, 0])


def test_planted_gqa_map_is_caught():
    w = workloads.prefill_config((12,), 8, 2, 16, seed=5)
    got = oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens,
                               w.scale)
    h = 1  # kv head 0 under h // G; kv head 1 under the planted h % Hkv
    K = w.key.astype(np.float64)[:, 1]
    V = w.value.astype(np.float64)[:, 1]
    sc = w.q[5, h].astype(np.float64) @ K[:6].T * w.scale
    p = np.exp(sc - sc.max())
    planted = (p / p.sum()) @ V[:6]
    assert not np.allclose(planted, got[5, h])
