"""Size-independent properties of attention, checked on the GPU's own outputs
at BASELINE sizes (configs 2 and 3), beside the oracle comparisons of
test_gpu_decode.py. Each follows from the definition out = sum_t w_t V[t]
with w = softmax(scale q.K^T) over the context, whatever the size:

  dominant key   all query heads of a kv group equal and one key 100x that
                 query: every other weight underflows to 0 in fp32, so the
                 output is that token's V row, bit for bit (the kept weight
                 cancels in the division by the row sum up to a few fp32
                 ulps, far inside half an fp16 ulp of an fp16 V element). A
                 token taken from the wrong slot of a block, or a wrong
                 block, gives another row.
  zero query     every score is 0, so the output is the mean of V over the
                 context (attention tolerance against the float64 mean)
  convex hull    the output is a convex combination of V rows, so each
                 element lies within [min_t V, max_t V] of its kv head and
                 dimension (within half an fp16 ulp)

Each runs v1, split-K at 512-token partitions and balanced mode. The
prefill test holds the causal mask to the same two kinds of check at config
9 size: prefix softmaxes (a query shared by a prompt's tokens) and a
dominant key that only the tokens from its position on may see.
"""

import numpy as np
import pytest

from helpers import DeviceWorkload, assert_attention_close
from swiftllm_amd import workloads
from swiftllm_amd._hip import synchronize

pytestmark = pytest.mark.gpu

MODES = (("v1", None), ("v2", 512), ("v2", 0))


def _gather_v(w, s):
    """V of sequence s over its context: [ctx, Hkv, D] (fp16)."""
    L = int(w.context_lens[s])
    t = np.arange(L)
    return w.value_cache[w.block_tables[s, t // 16], :, :, t % 16]


def test_dominant_key_selects_its_value_row(dev):
    w = workloads.decode_config(2, seed=31)
    rng = np.random.default_rng(31)
    S, H, D = w.q.shape
    Hkv = w.key_cache.shape[1]
    G = H // Hkv
    qk = (rng.standard_normal((S, Hkv, D)) * 0.5).astype(np.float16)
    w.q = np.repeat(qk, G, axis=1)
    ctx = w.context_lens
    # first token, last token, and positions inside and on the edges of blocks
    pos = rng.integers(0, ctx)
    pos[0], pos[1], pos[2], pos[3] = 0, ctx[1] - 1, 15, 16
    expect = np.empty((S, H, D), np.float16)
    for s in range(S):
        j = int(pos[s])
        b, o = w.block_tables[s, j // 16], j % 16
        w.key_cache[b, :, :, o] = (qk[s].astype(np.float32) * 100.0).astype(np.float16)
        expect[s] = np.repeat(w.value_cache[b, :, :, o], G, axis=0)
    dw = DeviceWorkload(w)
    for variant, ps in MODES:
        out = dw.run(variant, partition_size=ps)
        bad = np.argwhere(out.view(np.uint16) != expect.view(np.uint16))
        assert bad.size == 0, f"{variant} ps={ps}: {len(bad)} elements differ, first (s, h, d) {bad[0]}"


@pytest.fixture(scope="module")
def config3(dev):
    w = workloads.decode_config(3, seed=3)
    return w, DeviceWorkload(w)


def test_zero_query_gives_the_mean_of_v(config3):
    w, dw = config3
    S, H, D = w.q.shape
    G = H // w.key_cache.shape[1]
    ref = np.stack([np.repeat(_gather_v(w, s).astype(np.float64).mean(axis=0), G, axis=0)
                    for s in range(S)])
    dw.q.upload(np.zeros_like(w.q))
    try:
        for variant, ps in MODES:
            assert_attention_close(dw.run(variant, partition_size=ps), ref, f"q = 0, {variant} ps={ps}")
    finally:
        dw.q.upload(w.q)
        synchronize()


def test_output_within_the_value_hull(config3):
    w, dw = config3
    S, H, D = w.q.shape
    G = H // w.key_cache.shape[1]
    lo = np.empty((S, H, D), np.float32)
    hi = np.empty((S, H, D), np.float32)
    for s in range(S):
        v = _gather_v(w, s).astype(np.float32)
        lo[s] = np.repeat(v.min(axis=0), G, axis=0)
        hi[s] = np.repeat(v.max(axis=0), G, axis=0)
    # an output rounded to fp16 may pass a bound by half an ulp of the bound
    slack_lo = np.spacing(np.abs(lo).astype(np.float16)).astype(np.float32) / 2
    slack_hi = np.spacing(np.abs(hi).astype(np.float16)).astype(np.float32) / 2
    for variant, ps in MODES:
        out = dw.run(variant, partition_size=ps).astype(np.float32)
        assert np.isfinite(out).all()
        assert (out >= lo - slack_lo).all() and (out <= hi + slack_hi).all(), f"{variant} ps={ps}"


def test_prefill_causal_prefixes_and_a_dominant_key(dev):
    """Prefill at config 9 size (8 prompts of 2048 tokens, 32 query heads, 8
    kv heads). Every token of a prompt uses the same query u (per kv head, all
    G heads equal), so causal attention reduces to prefix sums over the
    prompt's keys: out_i = sum_{t <= i} e_t V_t / sum_{t <= i} e_t with
    e_t = exp(scale u.K_t), an O(L D) reference at full size. One key per
    prompt, at position j, is 100 u: tokens i >= j must return V_j bit for
    bit, tokens i < j (which must not see it) the prefix softmax over the
    other keys. A token that attends past itself fails one or the other."""
    from swiftllm_amd import paged_attention as pa
    from swiftllm_amd._hip import DeviceArray

    w = workloads.prefill_config((2048,) * 8, 32, 8, 128, seed=9)
    rng = np.random.default_rng(9)
    T, H, D = w.q.shape
    Hkv = w.key_cache.shape[1]
    G = H // Hkv
    lens = w.context_lens.astype(np.int64)
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]])
    u = (rng.standard_normal((len(lens), Hkv, D)) * 0.5).astype(np.float16)
    jpos = rng.integers(0, lens)
    jpos[:4] = [0, lens[1] - 1, 15, 16]
    q = np.empty_like(w.q)
    for s, (st, L) in enumerate(zip(starts, lens)):
        q[st:st + L] = np.repeat(u[s], G, axis=0)[None]
        t = st + int(jpos[s])
        big = (u[s].astype(np.float32) * 100.0).astype(np.float16)
        slot = int(w.slot_mapping[t])
        w.key_cache[slot // 16, :, :, slot % 16] = big
        w.key[t] = big
    out = DeviceArray((T, H, D), np.float16)
    out.fill_byte(0xFF)
    pa.launch_paged_prefill(out, DeviceArray.from_numpy(q), DeviceArray.from_numpy(w.key_cache),
                            DeviceArray.from_numpy(w.value_cache), DeviceArray.from_numpy(w.slot_mapping),
                            DeviceArray.from_numpy(w.context_lens), w.scale, len(lens), H, Hkv, D, 16,
                            int(lens.max()), num_blocks=w.key_cache.shape[0])
    synchronize()
    got = out.numpy()
    for s, (st, L) in enumerate(zip(starts, lens)):
        j = int(jpos[s])
        vj = np.repeat(w.value[st + j], G, axis=0)                    # [H, D]
        after = got[st + j:st + L]
        assert np.array_equal(after.view(np.uint16), np.broadcast_to(vj, after.shape).view(np.uint16)), \
            f"prompt {s}: tokens from {j} on must return V[{j}]"
        if j == 0:
            continue
        ref = np.empty((j, H, D))
        for g in range(Hkv):
            k = w.key[st:st + j, g].astype(np.float64)
            v = w.value[st:st + j, g].astype(np.float64)
            sc = (k @ u[s, g].astype(np.float64)) * w.scale
            e = np.exp(sc - sc.max())
            pref = np.cumsum(e[:, None] * v, axis=0) / np.cumsum(e)[:, None]
            ref[:, g * G:(g + 1) * G] = pref[:, None, :]
        assert_attention_close(got[st:st + j], ref, f"prompt {s}: tokens before {j}")
