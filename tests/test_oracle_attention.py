"""Pins for the decode oracle (oracle.decode_f64 / decode_numpy / decode_f32).

The reference has no numeric test for attention, so the oracle is pinned by
checks that do not restate its formula:
  * a library routine: torch's scaled_dot_product_attention (float64, CPU) on
    K/V gathered by index arithmetic written independently here;
  * closed forms: one token gives that token's V row; q = 0 (or scale 0)
    gives the mean of V; a dominant key gives its V row;
  * invariants: outputs are convex combinations of V rows; relabelling the
    physical blocks does not change the result; the GQA map h -> h // G;
  * the split-K rescale identity the GPU reduce relies on;
  * planted mistakes in the oracle (GQA map, scale, tile transpose,
    context off-by-one) that at least one pin must catch.
"""

import math

import numpy as np
import pytest

import oracle
from swiftllm_amd import workloads


def _small(seed, S=3, H=8, Hkv=2, D=64, ctx=(1, 37, 200), NB=40, std=1.0):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, np.int32)
    MB = int(max((ctx + 15) // 16))
    bt = np.zeros((S, MB), np.int32)
    perm = rng.permutation(NB)
    pos = 0
    for s in range(S):
        n = (ctx[s] + 15) // 16
        bt[s, :n] = perm[pos:pos + n]
        pos += n
    kc = (rng.standard_normal((NB, Hkv, D, 16)) * std).astype(np.float16)
    vc = (rng.standard_normal((NB, Hkv, D, 16)) * std).astype(np.float16)
    q = (rng.standard_normal((S, H, D)) * std).astype(np.float16)
    return q, kc, vc, bt, ctx


def _gather_independent(cache, bt_row, L):
    """Token j of a sequence, written from the element formula
    ((b * Hkv + h) * D + d) * BS + t of paged_attention.cu:85-93, 114-123,
    on the flattened cache (no reshapes shared with the oracle)."""
    NB, Hkv, D, BS = cache.shape
    flat = cache.reshape(-1)
    out = np.empty((Hkv, L, D), dtype=np.float64)
    d = np.arange(D)
    for j in range(L):
        b, t = int(bt_row[j // BS]), j % BS
        for h in range(Hkv):
            out[h, j] = flat[((b * Hkv + h) * D + d) * BS + t]
    return out


def test_c_and_numpy_oracles_agree():
    for seed in range(3):
        q, kc, vc, bt, ctx = _small(seed)
        a = oracle.decode_f64(q, kc, vc, bt, ctx, 0.125)
        b = oracle.decode_numpy(q, kc, vc, bt, ctx, 0.125)
        assert np.abs(a - b).max() < 1e-12


@pytest.mark.parametrize("H,Hkv,D", [(8, 8, 64), (8, 2, 64), (32, 8, 128), (16, 1, 128)])
def test_matches_torch_sdpa(H, Hkv, D):
    torch = pytest.importorskip("torch")
    q, kc, vc, bt, ctx = _small(H + D, H=H, Hkv=Hkv, D=D, ctx=(5, 64, 100))
    scale = 1.0 / math.sqrt(D)
    ref = oracle.decode_f64(q, kc, vc, bt, ctx, scale)
    G = H // Hkv
    for s in range(len(ctx)):
        L = int(ctx[s])
        K = torch.from_numpy(_gather_independent(kc, bt[s], L))          # [Hkv, L, D]
        V = torch.from_numpy(_gather_independent(vc, bt[s], L))
        K = K.repeat_interleave(G, dim=0)                                 # head h uses kv head h // G
        V = V.repeat_interleave(G, dim=0)
        Q = torch.from_numpy(q[s].astype(np.float64)).unsqueeze(1)        # [H, 1, D]
        O = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=scale)[:, 0]
        assert np.abs(O.numpy() - ref[s]).max() < 1e-10


def test_single_token_gives_its_value_row():
    q, kc, vc, bt, ctx = _small(5, ctx=(1, 1, 1))
    out = oracle.decode_f64(q, kc, vc, bt, ctx, 0.3)
    G = q.shape[1] // kc.shape[1]
    for s in range(3):
        v0 = vc[bt[s, 0], :, :, 0].astype(np.float64)
        assert np.array_equal(out[s], np.repeat(v0, G, axis=0))


@pytest.mark.parametrize("mode", ["q_zero", "scale_zero"])
def test_uniform_weights_give_the_mean(mode):
    q, kc, vc, bt, ctx = _small(6)
    scale = 0.2
    if mode == "q_zero":
        q = np.zeros_like(q)
    else:
        scale = 0.0
    out = oracle.decode_f64(q, kc, vc, bt, ctx, scale)
    G = q.shape[1] // kc.shape[1]
    for s in range(3):
        V = _gather_independent(vc, bt[s], int(ctx[s]))
        assert np.abs(out[s] - np.repeat(V.mean(axis=1), G, axis=0)).max() < 1e-12


def test_dominant_key_selects_its_value():
    q, kc, vc, bt, ctx = _small(7, ctx=(50, 50, 50))
    # token 17 of sequence 0, kv head 0, gets a key far along q[0, 0]
    b, t = bt[0, 17 // 16], 17 % 16
    kc = kc.copy()
    kc[b, 0, :, t] = (np.sign(q[0, 0].astype(np.float32)) * 60).astype(np.float16)
    out = oracle.decode_f64(q, kc, vc, bt, ctx, 1.0)
    assert np.abs(out[0, 0] - vc[b, 0, :, t].astype(np.float64)).max() < 1e-9


def test_output_is_a_convex_combination():
    q, kc, vc, bt, ctx = _small(8, std=2.0)
    out = oracle.decode_f64(q, kc, vc, bt, ctx, 0.4)
    G = q.shape[1] // kc.shape[1]
    for s in range(3):
        V = _gather_independent(vc, bt[s], int(ctx[s]))
        lo = np.repeat(V.min(axis=1), G, axis=0)
        hi = np.repeat(V.max(axis=1), G, axis=0)
        assert np.all(out[s] >= lo - 1e-12) and np.all(out[s] <= hi + 1e-12)


def test_block_relabelling_invariance():
    q, kc, vc, bt, ctx = _small(9)
    NB = kc.shape[0]
    perm = np.random.default_rng(1).permutation(NB)   # new id of old block b: perm[b]
    kc2 = np.empty_like(kc)
    vc2 = np.empty_like(vc)
    kc2[perm] = kc
    vc2[perm] = vc
    bt2 = perm[bt].astype(np.int32)
    a = oracle.decode_f64(q, kc, vc, bt, ctx, 0.125)
    b = oracle.decode_f64(q, kc2, vc2, bt2, ctx, 0.125)
    assert np.array_equal(a, b)


def test_gqa_map_is_head_div_group():
    """With kv head k holding constant K = 0 and V = k + 1, every query head h
    must read V = h // G + 1 (paged_attention.cu:52)."""
    S, H, Hkv, D = 2, 8, 2, 64
    q, kc, vc, bt, ctx = _small(10, S=S, H=H, Hkv=Hkv, D=D, ctx=(20, 33))
    kc = np.zeros_like(kc)
    for k in range(Hkv):
        vc[:, k] = k + 1
    out = oracle.decode_f64(q, kc, vc, bt, ctx, 0.125)
    for h in range(H):
        assert np.all(out[:, h] == h // (H // Hkv) + 1)


def test_fp32_baseline_matches_fp64():
    w = workloads.decode_config(1, seed=3)
    a = oracle.decode_f64(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)
    b = oracle.decode_f32(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)
    assert np.abs(a - b).max() < 1e-5


def test_fp32_baseline_gqa_and_tails():
    q, kc, vc, bt, ctx = _small(11, H=32, Hkv=8, D=128, ctx=(1, 15, 17, 160)[:3])
    a = oracle.decode_f64(q, kc, vc, bt, ctx, 1 / math.sqrt(128))
    b = oracle.decode_f32(q, kc, vc, bt, ctx, 1 / math.sqrt(128))
    assert np.abs(a - b).max() < 1e-5


def test_zero_context_gives_zeros():
    q, kc, vc, bt, ctx = _small(12, ctx=(0, 5, 0))
    for fn in (oracle.decode_f64, oracle.decode_f32, oracle.decode_numpy):
        out = fn(q, kc, vc, bt, ctx, 0.1)
        assert np.all(out[0] == 0) and np.all(out[2] == 0)


def test_split_k_rescale_identity():
    """Per-partition (m_p, l_p, o_p) combined with w_p = l_p exp(m_p - M)
    reproduce the single-pass result: the reduce the GPU's split-K kernel does."""
    rng = np.random.default_rng(13)
    L, D = 1000, 64
    logits = rng.standard_normal(L) * 3
    V = rng.standard_normal((L, D))
    p = np.exp(logits - logits.max())
    full = p @ V / p.sum()
    ms, ls, os_ = [], [], []
    for a in range(0, L, 96):
        z = logits[a:a + 96]
        m = z.max()
        e = np.exp(z - m)
        ms.append(m)
        ls.append(e.sum())
        os_.append(e @ V[a:a + 96] / e.sum())
    M = max(ms)
    w = np.array(ls) * np.exp(np.array(ms) - M)
    comb = (w[:, None] * np.array(os_)).sum(0) / w.sum()
    assert np.abs(comb - full).max() < 1e-12


# --- planted mistakes: each mutated oracle must fail at least one pin ---------

def test_planted_gqa_map_is_caught():
    S, H, Hkv, D = 2, 8, 2, 64
    q, kc, vc, bt, ctx = _small(10, S=S, H=H, Hkv=Hkv, D=D, ctx=(20, 33))
    kc = np.zeros_like(kc)
    for k in range(Hkv):
        vc[:, k] = k + 1
    wrong = oracle.decode_numpy(q, kc, vc, bt, ctx, 0.125, kv_head_of=lambda h, H, Hkv: h % Hkv)
    assert not all(np.all(wrong[:, h] == h // (H // Hkv) + 1) for h in range(H))


def test_planted_missing_scale_is_caught():
    torch = pytest.importorskip("torch")
    q, kc, vc, bt, ctx = _small(14, ctx=(40, 40, 40))
    wrong = oracle.decode_numpy(q, kc, vc, bt, ctx, 1.0)          # scale dropped
    L = 40
    K = torch.from_numpy(_gather_independent(kc, bt[0], L)).repeat_interleave(4, 0)
    V = torch.from_numpy(_gather_independent(vc, bt[0], L)).repeat_interleave(4, 0)
    Q = torch.from_numpy(q[0].astype(np.float64)).unsqueeze(1)
    O = torch.nn.functional.scaled_dot_product_attention(Q, K, V, scale=0.125)[:, 0].numpy()
    assert np.abs(O - wrong[0]).max() > 1e-3


def test_planted_tile_transpose_is_caught():
    """Reading the tile as [BS, D] instead of [D, BS] breaks the single-token pin."""
    q, kc, vc, bt, ctx = _small(15, ctx=(1, 1, 1))
    NB, Hkv, D, BS = vc.shape
    vc_wrong_view = vc.reshape(NB, Hkv, BS, D).transpose(0, 1, 3, 2).copy()  # mis-read layout
    out = oracle.decode_f64(q, kc, vc_wrong_view, bt, ctx, 0.3)
    v0 = vc[bt[0, 0], :, :, 0].astype(np.float64)
    assert not np.array_equal(out[0], np.repeat(v0, 4, axis=0))


def test_planted_context_off_by_one_is_caught():
    """Pin: with two tokens the output is a strict mixture of the two V rows,
    never the first row alone. An oracle that drops the last token fails it."""
    q, kc, vc, bt, ctx = _small(16, ctx=(2, 2, 2))
    v0 = np.repeat(vc[bt[0, 0], :, :, 0].astype(np.float64), 4, axis=0)
    good = oracle.decode_f64(q, kc, vc, bt, ctx, 0.3)
    assert not np.array_equal(good[0], v0)
    mutated = oracle.decode_f64(q, kc, vc, bt, ctx - 1, 0.3)   # drops the last token
    assert np.array_equal(mutated[0], v0)
