"""KV pools past 4 GiB: every path that addresses the cache, on blocks whose
element offsets pass 2^31 (and byte offsets 2^32), against the oracle on a
compact copy of the same blocks.

An MI355X holds 288 GB, so a serving pool of tens of GiB per cache is the
normal case, and a 32-bit product anywhere in a tile address would wrap
there while every small-pool test passes. The pool here is 200,000 blocks of
8 kv heads x 128 x 16 fp16 (32 KiB per block, 6.1 GiB per cache, 12.2 GiB in
all), filled with NaN; only the blocks a test uses are uploaded, so a read
of any other block shows up as NaN and a write to a wrong address leaves the
expected block unwritten. Block 131,072 is the first whose first element is
at offset 2^31; each test draws its blocks from its own range above it
(decode also takes the blocks on either side of that line, the last block of
the pool and a few low ones), so the tests can run in any order.

  decode       v1 (bounded), split-K at 512-token partitions, balanced, and
               the params-struct entry (unbounded): attention tolerance
  cache write  the launcher and the params-struct entry: bit-exact on the
               written blocks, slots crossing block boundaries, a -1 slot
  prefill      packed prompts of 1, 40 and 700 tokens: attention tolerance
  copy_blocks  high -> low, low -> high and high -> high pairs: bit-exact
"""

import numpy as np
import pytest

import oracle
from helpers import assert_attention_close
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu

NB = 200_000
HKV, D, H, BS = 8, 128, 32, 16
TILE = HKV * D * BS                  # fp16 elements per block
BLOCK_BYTES = 2 * TILE               # 32 KiB
FIRST_HIGH = (1 << 31) // TILE       # 131072: first element at offset 2^31
SCALE = 1.0 / np.sqrt(D)


@pytest.fixture(scope="module")
def pool(dev):
    kc = DeviceArray((NB, HKV, D, BS), np.float16)
    vc = DeviceArray((NB, HKV, D, BS), np.float16)
    kc.fill_byte(0xFF)
    vc.fill_byte(0xFF)
    synchronize()
    yield kc, vc
    kc.free()
    vc.free()


def _put_blocks(cache, ids, tiles):
    for b, t in zip(ids, tiles):
        cache.upload_at(int(b) * BLOCK_BYTES, t)


def _get_blocks(cache, ids):
    return np.stack([cache.download_at(int(b) * BLOCK_BYTES, (HKV, D, BS), np.float16) for b in ids])


def _fill_sequences(rng, pool, ctx, ids):
    """Uploads random K/V for the valid slots of each sequence's blocks
    (NaN past its context) and returns the block tables (real ids), the
    compact tables (0..n-1) and the compact K and V caches."""
    kc, vc = pool
    need = (ctx + BS - 1) // BS
    mb = int(need.max())
    bt = np.zeros((len(ctx), mb), np.int32)
    bt_c = np.zeros((len(ctx), mb), np.int32)
    n = int(need.sum())
    k_c = np.full((n, HKV, D, BS), np.nan, np.float16)
    v_c = np.full((n, HKV, D, BS), np.nan, np.float16)
    pos = 0
    for s, L in enumerate(ctx):
        for j in range(int(need[s])):
            valid = min(BS, int(L) - BS * j)
            k_c[pos, :, :, :valid] = rng.standard_normal((HKV, D, valid))
            v_c[pos, :, :, :valid] = rng.standard_normal((HKV, D, valid))
            bt[s, j], bt_c[s, j] = ids[pos], pos
            pos += 1
    _put_blocks(kc, ids[:n], k_c)
    _put_blocks(vc, ids[:n], v_c)
    return bt, bt_c, k_c, v_c


def test_decode_above_4gib(pool):
    kc, vc = pool
    rng = np.random.default_rng(71)
    ctx = np.array([1, 17, 300, 1000, 2500, 4096], np.int32)
    S = len(ctx)
    n = int(((ctx + BS - 1) // BS).sum())
    edge = [FIRST_HIGH - 1, FIRST_HIGH, NB - 1]
    low = rng.choice(1000, size=8, replace=False)
    high = rng.choice(np.arange(FIRST_HIGH + 1, 160_000), size=n - len(edge) - len(low), replace=False)
    ids = rng.permutation(np.concatenate([edge, low, high])).astype(np.int64)
    bt, bt_c, k_c, v_c = _fill_sequences(rng, pool, ctx, ids)
    assert (bt >= FIRST_HIGH).sum() > n // 2
    mb = bt.shape[1]
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    ref = oracle.decode_f64(q, k_c, v_c, bt_c, ctx, SCALE)
    qd, btd, ctxd = DeviceArray.from_numpy(q), DeviceArray.from_numpy(bt), DeviceArray.from_numpy(ctx)
    out = DeviceArray((S, H, D), np.float16)

    out.fill_byte(0xFF)
    pa.paged_attention_v1(out, qd, kc, vc, btd, ctxd, SCALE, S, H, HKV, D, BS, mb, num_blocks=NB)
    synchronize()
    assert_attention_close(out.numpy(), ref, "v1")
    for ps in (512, 0):
        need = pa.paged_attention_v2_workspace_size(S, H, HKV, D, BS, mb, ps)
        ws = pa.workspace(need)
        out.fill_byte(0xFF)
        pa.paged_attention_v2(out, ws, qd, kc, vc, btd, ctxd, SCALE, S, H, HKV, D, BS, mb, ps,
                              num_blocks=NB)
        synchronize()
        assert_attention_close(out.numpy(), ref, f"v2 partition {ps}")
    out.fill_byte(0xFF)
    params = pa.PagedAttentionParams(S, H, HKV, D, BS, SCALE, mb * BS)
    pa.paged_attention_decode(out, qd, kc, vc, btd, ctxd, params)
    synchronize()
    assert_attention_close(out.numpy(), ref, "params-struct decode")


@pytest.mark.parametrize("entry", ["launcher", "params"])
def test_cache_write_above_4gib(pool, entry):
    kc, vc = pool
    rng = np.random.default_rng(72 if entry == "launcher" else 73)
    lo_, hi_ = (160_000, 170_000) if entry == "launcher" else (170_000, 180_000)
    blocks = rng.choice(np.arange(lo_, hi_), size=6, replace=False).astype(np.int64)
    # runs of consecutive slots that cross from one block into the next, one
    # padding slot (-1) and single slots
    slots_c = np.concatenate([np.arange(10, 30), np.arange(3 * BS + 14, 5 * BS + 2), [-1],
                              [2 * BS + 7, 5 * BS + 15]]).astype(np.int32)
    slots = np.where(slots_c >= 0, blocks[np.maximum(slots_c, 0) // BS] * BS + slots_c % BS, -1)
    slots = slots.astype(np.int32)
    T = len(slots)
    key = rng.standard_normal((T, HKV, D)).astype(np.float16)
    value = rng.standard_normal((T, HKV, D)).astype(np.float16)
    k_c, v_c = _get_blocks(kc, blocks), _get_blocks(vc, blocks)
    oracle.reshape_and_cache(key, value, k_c, v_c, slots_c)
    kd, vd, sd = DeviceArray.from_numpy(key), DeviceArray.from_numpy(value), DeviceArray.from_numpy(slots)
    if entry == "launcher":
        pa.launch_reshape_and_cache(kd, vd, kc, vc, sd, T, HKV, D, BS, num_blocks=NB)
    else:
        pa.reshape_and_cache(kd, vd, kc, vc, sd, pa.ReshapeCacheParams(T, HKV, D, BS))
    synchronize()
    assert np.array_equal(_get_blocks(kc, blocks).view(np.uint16), k_c.view(np.uint16))
    assert np.array_equal(_get_blocks(vc, blocks).view(np.uint16), v_c.view(np.uint16))


def test_prefill_above_4gib(pool):
    kc, vc = pool
    rng = np.random.default_rng(74)
    ctx = np.array([1, 40, 700], np.int32)
    n = int(((ctx + BS - 1) // BS).sum())
    ids = rng.choice(np.arange(180_000, 190_000), size=n, replace=False).astype(np.int64)
    bt, bt_c, k_c, v_c = _fill_sequences(rng, pool, ctx, ids)
    sm, sm_c = [], []
    for s, L in enumerate(ctx):
        i = np.arange(int(L))
        sm.append(bt[s, i // BS].astype(np.int64) * BS + i % BS)
        sm_c.append(bt_c[s, i // BS] * BS + i % BS)
    sm = np.concatenate(sm).astype(np.int32)
    sm_c = np.concatenate(sm_c).astype(np.int32)
    T = int(ctx.sum())
    q = rng.standard_normal((T, H, D)).astype(np.float16)
    ref = oracle.prefill_numpy(q, k_c, v_c, sm_c, ctx, SCALE)
    out = DeviceArray((T, H, D), np.float16)
    out.fill_byte(0xFF)
    pa.launch_paged_prefill(out, DeviceArray.from_numpy(q), kc, vc, DeviceArray.from_numpy(sm),
                            DeviceArray.from_numpy(ctx), SCALE, len(ctx), H, HKV, D, BS,
                            int(ctx.max()), num_blocks=NB)
    synchronize()
    assert_attention_close(out.numpy(), ref, "prefill")


def test_copy_blocks_above_4gib(pool):
    kc, vc = pool
    rng = np.random.default_rng(75)
    high = rng.choice(np.arange(190_000, NB - 1), size=8, replace=False).astype(np.int64)
    low = rng.choice(np.arange(1000, 2000), size=4, replace=False).astype(np.int64)
    pairs = np.array([[high[0], low[0]], [high[1], low[1]],     # high -> low
                      [low[2], high[2]], [low[3], high[3]],     # low -> high
                      [high[4], high[5]], [high[6], high[7]]],  # high -> high
                     np.int64)
    src = pairs[:, 0]
    k_src = rng.standard_normal((len(src), HKV, D, BS)).astype(np.float16)
    v_src = rng.standard_normal((len(src), HKV, D, BS)).astype(np.float16)
    _put_blocks(kc, src, k_src)
    _put_blocks(vc, src, v_src)
    pa.launch_copy_blocks(DeviceArray.from_numpy(pairs), kc, vc, len(pairs), HKV, D, BS,
                          num_blocks=NB)
    synchronize()
    dst = pairs[:, 1]
    assert np.array_equal(_get_blocks(kc, dst).view(np.uint16), k_src.view(np.uint16))
    assert np.array_equal(_get_blocks(vc, dst).view(np.uint16), v_src.view(np.uint16))
    assert np.array_equal(_get_blocks(kc, src).view(np.uint16), k_src.view(np.uint16))
