"""Size-independent properties of attention, checked on the GPU's own outputs
at BASELINE sizes (configs 2 and 3), beside the oracle comparisons of
test_gpu_decode.py. Each follows from the definition out = sum_t w_t V[t]
with w = softmax(scale q.K^T) over the context, whatever the size:

  dominant key   all query heads of a kv group equal and one key 100x that
                 query: every other weight underflows to 0 in fp32, so the
                 output is that token's V row, bit for bit (the weight of the
                 kept token is a power of two, so the sum and the division by
                 the row sum are exact). A token taken from the wrong slot of
                 a block, or a wrong block, gives another row.
  zero query     every score is 0, so the output is the mean of V over the
                 context (attention tolerance against the float64 mean)
  convex hull    the output is a convex combination of V rows, so each
                 element lies within [min_t V, max_t V] of its kv head and
                 dimension (within half an fp16 ulp)

Each runs v1, split-K at 512-token partitions and balanced mode.
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
