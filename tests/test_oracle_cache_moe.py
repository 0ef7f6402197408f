"""Pins for the cache-write and MoE parts of the oracle.

reshape_and_cache (paged_attention.cu:167-199) is pinned by tagged values:
every written element carries its own (token, head, dim) code, so the
destination of each one is checked against the closed-form address, and a
write followed by the block-table gather returns the tokens that went in.

MoE routing / dispatch are pinned by brute force in plain Python loops on
small inputs (sorting by (-logit, index); collecting entries expert by
expert), by closed forms for the weights and by permutation invariants.
"""

import math

import numpy as np
import pytest

import oracle

SENT = np.uint16(0x7E01)


def _tagged(T, Hkv, D):
    t, h, d = np.meshgrid(np.arange(T), np.arange(Hkv), np.arange(D), indexing="ij")
    return ((t * 1000 + h * 100 + d) % 60000 + 1).astype(np.uint16)


@pytest.mark.parametrize("impl", ["c", "numpy"])
def test_reshape_and_cache_tagged_addresses(impl):
    T, Hkv, D, BS, NB = 40, 4, 32, 16, 12
    rng = np.random.default_rng(0)
    slots = rng.choice(NB * BS, size=T, replace=False).astype(np.int32)
    slots[::9] = -1
    key = _tagged(T, Hkv, D)
    value = key + np.uint16(7)
    kc = np.full((NB, Hkv, D, BS), SENT, np.uint16)
    vc = kc.copy()
    fn = oracle.reshape_and_cache if impl == "c" else oracle.reshape_and_cache_numpy
    fn(key, value, kc, vc, slots)
    flat_k = kc.reshape(-1)
    written = np.zeros(flat_k.size, bool)
    for t in range(T):
        if slots[t] < 0:
            continue
        b, o = divmod(int(slots[t]), BS)
        for h in range(Hkv):
            for d in range(D):
                addr = ((b * Hkv + h) * D + d) * BS + o          # cu:191 element address
                assert flat_k[addr] == key[t, h, d]
                assert vc.reshape(-1)[addr] == value[t, h, d]
                written[addr] = True
    assert np.all(flat_k[~written] == SENT)


def test_write_then_gather_round_trip():
    """Tokens written at the slots of a block table come back from the gather."""
    rng = np.random.default_rng(1)
    Hkv, D, BS, NB = 2, 16, 16, 10
    table = list(rng.permutation(NB)[:4])
    L = 50
    slots = np.array(oracle.slot_mapping(table, BS, 0, L), np.int32)
    key = rng.standard_normal((L, Hkv, D)).astype(np.float16)
    kc = np.zeros((NB, Hkv, D, BS), np.float16)
    vc = np.zeros_like(kc)
    oracle.reshape_and_cache(key, key, kc, vc, slots)
    got = oracle.gather_kv(kc, np.array(table), L)           # [Hkv, L, D]
    assert np.array_equal(got.transpose(1, 0, 2).view(np.uint16), key.view(np.uint16))


def test_planted_cache_transpose_is_caught():
    """Writing into a [NB, Hkv, BS, D] reading of the cache breaks the
    tagged-address pin."""
    T, Hkv, D, BS, NB = 8, 2, 32, 16, 4
    slots = np.arange(T, dtype=np.int32) * 3
    key = _tagged(T, Hkv, D)
    kc = np.full((NB, Hkv, BS, D), SENT, np.uint16)
    b, o = slots // BS, slots % BS
    kc[b, :, o, :] = key                                      # wrong layout
    flat = kc.reshape(-1)
    addr = ((b[1] * Hkv + 0) * D + 5) * BS + o[1]
    assert flat[addr] != key[1, 0, 5]


def _route_brute(logits, K):
    ids, ws = [], []
    for row in logits.astype(np.float64):
        order = sorted(range(len(row)), key=lambda e: (-row[e], e))[:K]
        m = max(row)
        e = [math.exp(row[i] - m) for i in order]
        ids.append(order)
        ws.append([x / sum(e) for x in e])
    return np.array(ids, np.int32), np.array(ws)


@pytest.mark.parametrize("T,E,K", [(37, 8, 2), (20, 16, 4), (9, 5, 5), (30, 64, 8)])
def test_route_matches_brute_force(T, E, K):
    rng = np.random.default_rng(T + E)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, :3] = logits[0, E - 1]                           # ties
    ids, w = oracle.moe_route(logits, K)
    bids, bw = _route_brute(logits, K)
    assert np.array_equal(ids, bids)
    assert np.abs(w - bw).max() < 1e-15


def test_route_weight_closed_forms():
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((50, 8)).astype(np.float32)
    ids, w = oracle.moe_route(logits, 2)
    assert np.allclose(w.sum(1), 1.0, atol=1e-15)
    x = np.take_along_axis(logits.astype(np.float64), ids.astype(np.int64), 1)
    # w0 / w1 = exp(x0 - x1); for top-2, w0 = sigmoid(x0 - x1)
    assert np.allclose(w[:, 0] / w[:, 1], np.exp(x[:, 0] - x[:, 1]), rtol=1e-13)
    assert np.allclose(w[:, 0], 1 / (1 + np.exp(x[:, 1] - x[:, 0])), rtol=1e-13)
    assert np.all(x[:, 0] >= x[:, 1])


def test_route_ties_keep_lower_index():
    """sampling/mod.rs:374 sorts stably by descending logit."""
    logits = np.zeros((1, 8), np.float32)
    ids, w = oracle.moe_route(logits, 3)
    assert ids[0].tolist() == [0, 1, 2]
    assert np.allclose(w, 1 / 3)


def test_planted_unstable_ties_are_caught():
    logits = np.zeros((1, 8), np.float32)
    unstable = np.argsort(-logits, axis=1, kind="quicksort")[:, ::-1][:, :3]  # reversed ties
    assert unstable[0].tolist() != _route_brute(logits, 3)[0][0].tolist()


def _dispatch_brute(ids, E):
    T, K = ids.shape
    rows, counts = [], []
    for e in range(E):
        entries = [(t, k) for t in range(T) for k in range(K) if ids[t, k] == e]
        counts.append(len(entries))
        rows.extend(entries)
    inverse = np.full((T, K), -1, np.int32)
    for r, (t, k) in enumerate(rows):
        inverse[t, k] = r
    return np.array(counts, np.int32), inverse, np.array([t for t, _ in rows], np.int32)


@pytest.mark.parametrize("T,E,K", [(64, 8, 2), (100, 3, 3), (7, 16, 1), (130, 8, 4)])
def test_dispatch_matches_brute_force(T, E, K):
    rng = np.random.default_rng(T * E)
    ids = rng.integers(0, E, size=(T, K)).astype(np.int32)
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, E)
    bc, binv, bsorted = _dispatch_brute(ids, E)
    assert np.array_equal(counts, bc)
    assert np.array_equal(inverse, binv)
    assert np.array_equal(sorted_ids, bsorted)
    assert offsets[0] == 0 and offsets[-1] == T * K and np.all(np.diff(offsets) == counts)
    # inverse is a bijection onto the rows and sends every entry to its expert's range
    assert sorted(inverse.reshape(-1).tolist()) == list(range(T * K))
    for t in range(T):
        for k in range(K):
            r = inverse[t, k]
            assert sorted_ids[r] == t
            assert offsets[ids[t, k]] <= r < offsets[ids[t, k] + 1]


@pytest.mark.parametrize("T,E,K,hidden", [(64, 8, 2, 64), (37, 16, 4, 8), (9, 5, 5, 16),
                                          (130, 64, 8, 24)])
def test_serial_route_dispatch_matches_brute_force(T, E, K, hidden):
    """The one-thread C route + counting sort (the MoE CPU baseline) against
    the brute-force sort of the logits and the brute-force collection of
    entries per expert: ids, counts, offsets, inverse, sorted ids and the
    permuted rows bit-exact, fp32 weights within 1e-6 of fp64."""
    rng = np.random.default_rng(T + E + K)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    logits[0, :3] = logits[0, E - 1]                           # ties
    logits[1, :] = 0.0                                         # all tied
    x = rng.standard_normal((T, hidden)).astype(np.float16)
    ids, w, counts, offsets, x_perm, inverse, sorted_ids = oracle.moe_route_dispatch_serial(logits, x, K)
    bids, bw = _route_brute(logits, K)
    assert np.array_equal(ids, bids)
    assert np.abs(w - bw).max() < 1e-6
    bc, binv, bsorted = _dispatch_brute(bids, E)
    assert np.array_equal(counts, bc)
    assert np.array_equal(offsets, np.concatenate([[0], np.cumsum(bc)]))
    assert np.array_equal(inverse, binv)
    assert np.array_equal(sorted_ids, bsorted)
    assert np.array_equal(x_perm.view(np.uint16), x[bsorted].view(np.uint16))


def test_planted_unstable_placement_is_caught():
    """Placing entries in (k, t) order instead of (t, k) changes the rows."""
    ids = np.array([[0, 1], [1, 0], [0, 1]], np.int32)
    _, binv, _ = _dispatch_brute(ids, 2)
    rows, fill = np.empty_like(binv), [0, 3]
    for k in range(2):
        for t in range(3):
            rows[t, k] = fill[ids[t, k]]
            fill[ids[t, k]] += 1
    assert not np.array_equal(rows, binv)


def test_dispatch_drops_out_of_range_ids():
    ids = np.array([[0, -1], [5, 1], [1, 0]], np.int32)
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, 4)
    assert counts.tolist() == [2, 2, 0, 0]
    assert inverse.tolist() == [[0, -1], [-1, 2], [3, 1]]
    assert sorted_ids.tolist() == [0, 2, 1, 2]


def _tagged_pool(NB, Hkv, D, BS, salt):
    b, h, d, t = np.meshgrid(np.arange(NB), np.arange(Hkv), np.arange(D), np.arange(BS),
                             indexing="ij")
    return ((b * 7919 + h * 211 + d * 17 + t + salt) % 65000 + 1).astype(np.uint16)


def test_copy_blocks_tagged_pool():
    """Every element of a destination block carries the tag of the same
    (head, d, t) in its source block; every other block keeps its own tags."""
    NB, Hkv, D, BS = 12, 2, 32, 16
    layers = 3
    kcs = [_tagged_pool(NB, Hkv, D, BS, 100 * l) for l in range(layers)]
    vcs = [_tagged_pool(NB, Hkv, D, BS, 100 * l + 50) for l in range(layers)]
    before_k = [k.copy() for k in kcs]
    before_v = [v.copy() for v in vcs]
    mapping = np.array([[1, 7], [4, 9], [-1, 3], [2, 11]], np.int64)
    oracle.copy_blocks(kcs, vcs, mapping)
    moved = {7: 1, 9: 4, 11: 2}
    for l in range(layers):
        for b in range(NB):
            src = moved.get(b, b)
            assert np.array_equal(kcs[l][b], before_k[l][src])
            assert np.array_equal(vcs[l][b], before_v[l][src])


def test_planted_swapped_pair_order_is_caught():
    """Reading the pair as (dst, src) moves the wrong block."""
    NB, Hkv, D, BS = 6, 1, 16, 16
    kc = _tagged_pool(NB, Hkv, D, BS, 0)
    ref = kc.copy()
    oracle.copy_blocks([ref], [], np.array([[1, 4]], np.int64))
    planted = kc.copy()
    planted[1] = planted[4]
    assert not np.array_equal(planted, ref)


def test_swap_blocks_matches_byte_loop():
    rng = np.random.default_rng(7)
    nbytes, NS, ND = 40, 9, 6
    src = rng.integers(0, 256, size=NS * nbytes, dtype=np.uint8)
    dst = rng.integers(0, 256, size=ND * nbytes, dtype=np.uint8)
    mapping = np.array([[8, 0], [3, 5], [0, -1], [5, 2]], np.int64)
    expect = dst.copy()
    for a, b in mapping:
        if a >= 0 and b >= 0:
            for i in range(nbytes):
                expect[b * nbytes + i] = src[a * nbytes + i]
    oracle.swap_blocks(src, dst, mapping, nbytes)
    assert np.array_equal(dst, expect)


def test_silu_reference_kats_and_identities():
    """mlp.rs:313-317 (test_activation_silu): silu(0) = 0, silu(1) > 0.7,
    silu(-1) < -0.2; and silu(x) - silu(-x) = x, silu(x) = x * sigmoid(x)."""
    assert abs(oracle.silu(0.0)) < 1e-6
    assert oracle.silu(1.0) > 0.7
    assert oracle.silu(-1.0) < -0.2
    x = np.linspace(-20, 20, 81)
    assert np.allclose(oracle.silu(x) - oracle.silu(-x), x, atol=1e-12)
    assert np.allclose(oracle.silu(x), x * (0.5 * (1 + np.tanh(x / 2))), atol=1e-12)


def _expert_gemm_brute(a, w, w2, offsets):
    m, n = a.shape[0], w.shape[1]
    out = np.zeros((m, n))
    for e in range(w.shape[0]):
        for r in range(int(offsets[e]), int(offsets[e + 1])):
            for j in range(n):
                g = sum(float(a[r, q]) * float(w[e, j, q]) for q in range(a.shape[1]))
                if w2 is not None:
                    u = sum(float(a[r, q]) * float(w2[e, j, q]) for q in range(a.shape[1]))
                    g = g / (1 + math.exp(-g)) * u
                out[r, j] = g
    return out


@pytest.mark.parametrize("gated", [False, True])
def test_expert_gemm_matches_brute_force(gated):
    rng = np.random.default_rng(11 + gated)
    E, n, k = 3, 5, 7
    offsets = np.array([0, 4, 4, 9], np.int32)          # expert 1 has no rows
    a = rng.standard_normal((9, k)).astype(np.float16)
    w = rng.standard_normal((E, n, k)).astype(np.float16)
    w2 = rng.standard_normal((E, n, k)).astype(np.float16) if gated else None
    got = oracle.moe_expert_gemm(a, w, w2, offsets)
    assert np.allclose(got, _expert_gemm_brute(a, w, w2, offsets), atol=1e-12)


def test_planted_expert_off_by_one_is_caught():
    rng = np.random.default_rng(12)
    offsets = np.array([0, 3, 6], np.int32)
    a = rng.standard_normal((6, 4)).astype(np.float16)
    w = rng.standard_normal((2, 3, 4)).astype(np.float16)
    good = oracle.moe_expert_gemm(a, w, None, offsets)
    planted = oracle.moe_expert_gemm(a, w, None, np.array([0, 4, 6], np.int32))
    assert not np.allclose(good, planted)


def test_combine_matches_brute_force():
    rng = np.random.default_rng(13)
    T, K, hidden = 6, 3, 5
    y = rng.standard_normal((T * K, hidden)).astype(np.float16)
    w = rng.random((T, K)).astype(np.float32)
    inv = rng.permutation(T * K).reshape(T, K).astype(np.int32)
    inv[2, 1] = -1
    got = oracle.moe_combine(y, w, inv)
    for t in range(T):
        for d in range(hidden):
            ref = sum(float(w[t, k]) * float(y[inv[t, k], d]) for k in range(K) if inv[t, k] >= 0)
            assert abs(got[t, d] - ref) < 1e-12
