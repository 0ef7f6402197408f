"""Seeded random sweeps of the GPU paths against the oracle, beside the
hand-picked cases of the other test files: each case draws its shape (batch,
context lengths, heads and kv heads, head_dim, partition size, scale sign,
experts, top-k) from a fixed seed, so a failure names a case that can be
rerun exactly.

  decode   v1, v2 at a random partition size (multiple of 16), v2 balanced:
           attention tolerance against oracle.decode_f64, NaN in every cache
           slot outside the valid contexts, zero-length contexts giving zeros
  prefill  packed prompts of random lengths, positive and negative scales
           (the folded and the unfolded softmax): attention tolerance against
           oracle.prefill_numpy, NaN in unused slots
  moe      route + dispatch: expert ids, counts, offsets, inverse index,
           sorted ids and permuted rows bit-exact, weights within 1e-6
  experts  the grouped expert GEMM, plain and gated, over random expert
           counts (empty experts and 1-row tails included): the GEMM
           tolerance against oracle.moe_expert_gemm

Tolerances (tests/helpers.py): attention, max abs error <= 2e-3 and max
relative error <= 1e-2 with a 1e-3 floor on |ref|; expert GEMM, |gpu - ref| <=
2^-10 |ref| + 1e-3 rms(ref).
"""

import dataclasses

import numpy as np
import pytest

import oracle
from helpers import DeviceWorkload, assert_attention_close, assert_gemm_close, expert_offsets
from swiftllm_amd import moe
from swiftllm_amd import paged_attention as pa
from swiftllm_amd import workloads
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu

GQA = [(8, 8), (32, 8), (64, 8), (12, 4), (24, 2), (32, 1), (16, 1), (6, 3), (40, 8)]


def _decode_case(seed):
    rng = np.random.default_rng(seed)
    H, Hkv = GQA[rng.integers(len(GQA))]
    D = int(rng.choice([64, 128]))
    S = int(rng.integers(1, 25))
    kind = rng.integers(3)
    if kind == 0:
        ctx = rng.integers(0, 2049, S)
    elif kind == 1:  # lengths on block and partition edges
        ctx = rng.choice([0, 1, 15, 16, 17, 511, 512, 513, 1024, 2047], S)
    else:  # one long sequence among short ones
        ctx = rng.integers(0, 64, S)
        ctx[rng.integers(S)] = rng.integers(2048, 6000)
    ctx = ctx.astype(np.int32)
    need = (ctx + 15) // 16
    pad = int(rng.integers(0, 4))  # table columns past every sequence's last block
    MB = int(max(need.max(), 1)) + pad
    NB = int(need.sum()) + 5
    perm = rng.permutation(NB)
    bt = np.zeros((S, MB), np.int32)
    kc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    vc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    pos = 0
    for s in range(S):
        n = int(need[s])
        bt[s, :n] = perm[pos:pos + n]
        pos += n
        for j in range(n):
            valid = min(16, int(ctx[s]) - 16 * j)
            kc[bt[s, j], :, :, :valid] = rng.standard_normal((Hkv, D, valid)).astype(np.float16)
            vc[bt[s, j], :, :, :valid] = rng.standard_normal((Hkv, D, valid)).astype(np.float16)
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    ps = 16 * int(rng.integers(1, 65))
    w = workloads.DecodeWorkload(f"sweep{seed}", q, kc, vc, bt, ctx, 1.0 / np.sqrt(D))
    return w, ps


@pytest.mark.parametrize("seed", range(48))
def test_decode_random(dev, seed):
    w, ps = _decode_case(1000 + seed)
    ref = oracle.decode_f64(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)
    dw = DeviceWorkload(w)
    S, H, D = w.q.shape
    Hkv = w.key_cache.shape[1]
    what = f"seed {1000 + seed}: S={S} H={H} Hkv={Hkv} D={D} max ctx {int(w.context_lens.max())}"
    for variant, p in (("v1", None), ("v2", ps), ("v2", 0)):
        out = dw.run(variant, partition_size=p)
        assert np.all(out[w.context_lens == 0] == 0), f"{what} {variant} ps={p}: zero contexts"
        assert_attention_close(out, ref, f"{what} {variant} ps={p}")


@pytest.mark.parametrize("seed", range(16))
def test_prefill_random(dev, seed):
    rng = np.random.default_rng(2000 + seed)
    H, Hkv = GQA[rng.integers(len(GQA))]
    D = int(rng.choice([64, 128]))
    n = int(rng.integers(1, 7))
    lens = rng.integers(1, 300, n)
    if rng.integers(2):
        lens[rng.integers(n)] = rng.integers(300, 700)
    w = workloads.prefill_config(tuple(int(x) for x in lens), H, Hkv, D, seed=3000 + seed)
    if rng.integers(3) == 0:
        w = dataclasses.replace(w, scale=-w.scale)  # the unfolded softmax path
    T = w.q.shape[0]
    S = len(w.context_lens)
    out = DeviceArray((T, H, D), np.float16)
    out.fill_byte(0xFF)
    q = DeviceArray.from_numpy(w.q)
    kc, vc = DeviceArray.from_numpy(w.key_cache), DeviceArray.from_numpy(w.value_cache)
    sm, ctx = DeviceArray.from_numpy(w.slot_mapping), DeviceArray.from_numpy(w.context_lens)
    pa.launch_paged_prefill(out, q, kc, vc, sm, ctx, w.scale, S, H, Hkv, D, 16, int(w.context_lens.max()),
                            num_blocks=w.key_cache.shape[0])
    synchronize()
    ref = oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens, w.scale)
    assert_attention_close(out.numpy(), ref,
                           f"seed {2000 + seed}: lens {list(map(int, lens))} H={H} Hkv={Hkv} D={D} "
                           f"scale {w.scale:+.4f}")


@pytest.mark.parametrize("seed", range(20))
def test_moe_route_dispatch_random(dev, seed):
    rng = np.random.default_rng(4000 + seed)
    E = int(rng.choice([2, 3, 8, 16, 60, 128, 256]))
    K = int(rng.integers(1, min(E, 8) + 1))
    T = int(rng.choice([1, 2, 63, 64, 65, 500, 3000]))
    hidden = 8 * int(rng.integers(1, 65))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    if rng.integers(2):  # coarse logits: many ties
        logits = np.round(logits * 2) / 2
    x = rng.standard_normal((T, hidden)).astype(np.float16)
    what = f"seed {4000 + seed}: T={T} E={E} K={K} hidden={hidden}"
    rids, rw = oracle.moe_route(logits, K)
    ids = DeviceArray((T, K), np.int32)
    w = DeviceArray((T, K), np.float32)
    bufs = moe.DispatchBuffers.allocate(T, E, K, hidden, with_rows=True)
    bufs.workspace.fill_byte(0xFF)
    moe.moe_route_dispatch(DeviceArray.from_numpy(logits), DeviceArray.from_numpy(x), K, ids, w, bufs)
    synchronize()
    assert np.array_equal(ids.numpy(), rids), what
    assert np.abs(w.numpy() - rw).max() <= 1e-6, what
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(rids, E)
    assert np.array_equal(bufs.counts.numpy(), counts), what
    assert np.array_equal(bufs.offsets.numpy(), offsets), what
    assert np.array_equal(bufs.inverse.numpy(), inverse), what
    nrows = int(offsets[-1])
    assert np.array_equal(bufs.sorted_token_ids.numpy()[:nrows], sorted_ids), what
    assert np.array_equal(bufs.x_perm.numpy()[:nrows].view(np.uint16), x[sorted_ids].view(np.uint16)), what


@pytest.mark.parametrize("seed", range(12))
def test_expert_gemm_random(dev, seed):
    rng = np.random.default_rng(5000 + seed)
    gated = bool(rng.integers(2))
    E = int(rng.integers(1, 13))
    m_total = int(rng.choice([1, 255, 257, 700, 1500]))
    n = (128 if gated else 256) * int(rng.integers(1, 5))
    k = 64 * int(rng.integers(1, 17))
    empty = tuple(int(e) for e in rng.choice(E, size=min(E - 1, int(rng.integers(0, 3))), replace=False))
    offs = expert_offsets(rng, E, m_total, empty=empty)
    a = (rng.standard_normal((m_total, k)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16)
    w2 = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16) if gated else None
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(DeviceArray.from_numpy(a), DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None, DeviceArray.from_numpy(offs), c)
    synchronize()
    assert_gemm_close(c.numpy(), oracle.moe_expert_gemm(a, w, w2, offs),
                      f"seed {5000 + seed}: gated={gated} E={E} rows={m_total} n={n} k={k} "
                      f"counts {list(np.diff(offs))}")
