"""Paged-attention decode on the GPU against the fp64 C oracle.

Tolerance (fp16 in/out, fp32 accumulation): max abs error <= 2e-3 and max
relative error <= 1e-2 with a 1e-3 floor on |ref| (tests/helpers.py).
Index work (the block-table gather) is checked bit-exact.
"""

import numpy as np
import pytest

import oracle
from helpers import DeviceWorkload, assert_attention_close
from swiftllm_amd import paged_attention as pa
from swiftllm_amd import workloads
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def _ref(w):
    return oracle.decode_f64(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens, w.scale)


@pytest.mark.parametrize("variant,ps", [("v1", None), ("v2", 64), ("v2", 512), ("v2", 0), ("decode", None)])
def test_config1_tiny_mha(dev, variant, ps):
    w = workloads.decode_config(1, seed=11)
    out = DeviceWorkload(w).run(variant, partition_size=ps)
    assert_attention_close(out, _ref(w), f"config1 {variant} ps={ps}")


# 512: one wave per partition; 1024: two; 2048: the whole 4-wave workgroup
@pytest.mark.parametrize("variant,ps", [("v1", None), ("v2", 512), ("v2", 1024), ("v2", 2048),
                                        ("v2", 0)])
def test_config2_llama3_8b(dev, variant, ps):
    w = workloads.decode_config(2, seed=2)
    out = DeviceWorkload(w).run(variant, partition_size=ps)
    assert_attention_close(out, _ref(w), f"config2 {variant} ps={ps}")


def test_config3_long_context_split_k(dev):
    # Llama-3-70B layer, 64 partitions of 512 tokens per sequence, one x8
    # outlier key channel per kv head.
    w = workloads.decode_config(3, seed=3)
    dw = DeviceWorkload(w)
    ref = _ref(w)
    out = dw.run("v2", partition_size=512)
    assert_attention_close(out, ref, "config3 v2/512")
    # single pass and balanced scheduling agree with the oracle as well
    assert_attention_close(dw.run("v1"), ref, "config3 v1")
    assert_attention_close(dw.run("v2", partition_size=0), ref, "config3 balanced")
    for ps in (1024, 4096):
        assert_attention_close(dw.run("v2", partition_size=ps), ref, f"config3 v2/{ps}")


def test_config4_ragged_step(dev):
    """reshape_and_cache of the new tokens, then decode over the updated cache."""
    w = workloads.decode_config(4, seed=4)
    dw = DeviceWorkload(w)
    sh = w.shape
    k_new = DeviceArray.from_numpy(w.new_key)
    v_new = DeviceArray.from_numpy(w.new_value)
    sm = DeviceArray.from_numpy(w.slot_mapping)
    pa.launch_reshape_and_cache(k_new, v_new, dw.kc, dw.vc, sm, sh["num_seqs"], sh["num_kv_heads"],
                                sh["head_dim"], sh["block_size"], num_blocks=sh["num_blocks"])
    synchronize()
    kc_ref, vc_ref = w.key_cache.copy(), w.value_cache.copy()
    oracle.reshape_and_cache(w.new_key, w.new_value, kc_ref, vc_ref, w.slot_mapping)
    assert np.array_equal(dw.kc.numpy().view(np.uint16), kc_ref.view(np.uint16))
    assert np.array_equal(dw.vc.numpy().view(np.uint16), vc_ref.view(np.uint16))
    ref = oracle.decode_f64(w.q, kc_ref, vc_ref, w.block_tables, w.context_lens, w.scale)
    for variant, ps in (("v2", 512), ("v2", 0), ("v1", None)):
        assert_attention_close(dw.run(variant, partition_size=ps), ref, f"config4 {variant} ps={ps}")


@pytest.mark.parametrize("H,Hkv", [(8, 8), (16, 8), (32, 8), (64, 8), (16, 1), (32, 1), (48, 2)])
@pytest.mark.parametrize("D", [64, 128])
def test_gqa_groups(dev, H, Hkv, D):
    """G = 1, 2, 4, 8, 16, 32 (two 16-head chunks) and 24 (a ragged chunk)."""
    rng = np.random.default_rng(H * 1000 + Hkv * 10 + D)
    S = 3
    ctx = np.array([1, 37, 300], np.int32)
    NB = 40
    bt = np.zeros((S, 20), np.int32)
    perm = rng.permutation(NB)
    pos = 0
    for s in range(S):
        n = (ctx[s] + 15) // 16
        bt[s, :n] = perm[pos:pos + n]
        pos += n
    kc = rng.standard_normal((NB, Hkv, D, 16)).astype(np.float16)
    vc = rng.standard_normal((NB, Hkv, D, 16)).astype(np.float16)
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    w = workloads.DecodeWorkload("gqa", q, kc, vc, bt, ctx, 1.0 / np.sqrt(D))
    dw = DeviceWorkload(w)
    ref = _ref(w)
    for variant, ps in (("v1", None), ("v2", 32), ("v2", 0)):
        assert_attention_close(dw.run(variant, partition_size=ps), ref, f"H{H} Hkv{Hkv} D{D} {variant} ps={ps}")


def _poisoned(rng, S, ctx, D=128, H=32, Hkv=8, MB=None):
    """Caches whose every slot outside the valid context holds NaN."""
    need = (ctx + 15) // 16
    NB = int(need.sum()) + 3
    MB = MB or int(max(need.max(), 1))
    bt = np.zeros((S, MB), np.int32)
    perm = rng.permutation(NB)
    pos = 0
    kc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    vc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    for s in range(S):
        n = need[s]
        bt[s, :n] = perm[pos:pos + n]
        pos += n
        for j in range(n):
            valid = min(16, ctx[s] - 16 * j)
            kc[bt[s, j], :, :, :valid] = rng.standard_normal((Hkv, D, valid)).astype(np.float16)
            vc[bt[s, j], :, :, :valid] = rng.standard_normal((Hkv, D, valid)).astype(np.float16)
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    return workloads.DecodeWorkload("poison", q, kc, vc, bt, ctx.astype(np.int32), 1.0 / np.sqrt(D))


@pytest.mark.parametrize("variant,ps", [("v1", None), ("v2", 16), ("v2", 48), ("v2", 0)])
def test_edge_context_lengths(dev, variant, ps):
    """ctx in {0, 1, 15, 16, 17, 31, 33, 200}; unused slots hold NaN."""
    rng = np.random.default_rng(7)
    ctx = np.array([0, 1, 15, 16, 17, 31, 33, 200], np.int32)
    w = _poisoned(rng, len(ctx), ctx)
    out = DeviceWorkload(w).run(variant, partition_size=ps)
    ref = _ref(w)
    assert np.all(out[0] == 0), "context 0 must give zeros"
    # a single token: softmax weight 1, so the output is that token's V row exactly
    v0 = w.value_cache[w.block_tables[1, 0], :, :, 0]            # [Hkv, D]
    G = w.q.shape[1] // w.key_cache.shape[1]
    assert np.array_equal(out[1].view(np.uint16), np.repeat(v0, G, axis=0).view(np.uint16))
    assert_attention_close(out, ref, f"edge {variant} ps={ps}")


def test_out_of_pool_blocks_skipped(dev):
    """Block ids outside [0, num_blocks) contribute nothing; a sequence with
    no valid block yields zeros. (Only with the bounded entry points.)"""
    rng = np.random.default_rng(8)
    w = workloads.decode_config(1, seed=8)
    NB = w.key_cache.shape[0]
    bt = w.block_tables.copy()
    n0 = (w.context_lens[0] + 15) // 16
    bt[0, :n0] = NB + 1000 + rng.integers(0, 5, n0)
    w.block_tables = bt
    for variant, ps in (("v1", None), ("v2", 32), ("v2", 0)):
        out = DeviceWorkload(w).run(variant, partition_size=ps)
        assert np.all(out[0] == 0)
        ref = _ref(w)
        assert_attention_close(out[1:], ref[1:], f"oob {variant}")


@pytest.mark.parametrize("ps", [256, 0])
def test_deterministic(dev, ps):
    w = workloads.decode_config(2, seed=5, num_seqs=8)
    dw = DeviceWorkload(w)
    a = dw.run("v2", partition_size=ps).view(np.uint16)
    b = dw.run("v2", partition_size=ps).view(np.uint16)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("ps", [128, 0])
def test_workspace_reuse_across_shapes(dev, ps):
    """The split-K workspace is plain scratch: one buffer serves calls of
    different shapes in a row."""
    ws = pa.workspace(pa.paged_attention_v2_workspace_size(16, 32, 8, 128, 16, 256, ps))
    for seed, S, ctx in ((1, 16, 4000), (2, 5, 700), (3, 16, 1500)):
        w = workloads.decode_config(2, seed=seed, num_seqs=S, ctx=ctx)
        dw = DeviceWorkload(w)
        dw._ws = ws
        assert_attention_close(dw.run("v2", partition_size=ps), _ref(w), f"reuse S{S} ctx{ctx} ps={ps}")


def test_gather_bit_exact(dev):
    """The block-table gather (cu:80-87, 114-116) through the library's tile
    addressing equals the numpy gather bit for bit."""
    w = workloads.decode_config(1, seed=21)
    dw = DeviceWorkload(w)
    sh = w.shape
    Lmax = int(w.context_lens.max()) + 5
    D = sh["head_dim"]
    for s in range(sh["num_seqs"]):
        for kvh in (0, sh["num_kv_heads"] - 1):
            ko = DeviceArray((Lmax, D), np.float16)
            vo = DeviceArray((Lmax, D), np.float16)
            pa.gather_kv(dw.kc, dw.vc, dw.bt, dw.ctx, s, kvh, sh["num_kv_heads"], D, 16,
                         sh["max_num_blocks_per_seq"], Lmax, ko, vo)
            synchronize()
            L = int(w.context_lens[s])
            kr = oracle.gather_kv(w.key_cache, w.block_tables[s], L)[kvh]
            vr = oracle.gather_kv(w.value_cache, w.block_tables[s], L)[kvh]
            kg, vg = ko.numpy(), vo.numpy()
            assert np.array_equal(kg[:L].view(np.uint16), kr.view(np.uint16))
            assert np.array_equal(vg[:L].view(np.uint16), vr.view(np.uint16))
            assert np.all(kg[L:].view(np.uint16) == 0)


def test_dropin_launchers(dev):
    """The void launchers with the reference's argument lists."""
    from swiftllm_amd import _lib

    w = workloads.decode_config(1, seed=31)
    dw = DeviceWorkload(w)
    sh = w.shape
    L = _lib.lib()
    dw.out.fill_byte(0xFF)
    L.launch_paged_attention_v1(dw.out.ptr, dw.q.ptr, dw.kc.ptr, dw.vc.ptr, dw.bt.ptr, dw.ctx.ptr,
                                w.scale, sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"],
                                sh["head_dim"], sh["block_size"], sh["max_num_blocks_per_seq"], None)
    synchronize()
    assert L.swiftllm_hip_last_error() == 0
    assert_attention_close(dw.out.numpy(), _ref(w), "launch_paged_attention_v1")
    ws = pa.workspace(L.swiftllm_hip_paged_attention_v2_workspace_size(
        sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"], 16,
        sh["max_num_blocks_per_seq"], 64))
    dw.out.fill_byte(0xFF)
    L.launch_paged_attention_v2(dw.out.ptr, ws.ptr, ws.nbytes, dw.q.ptr, dw.kc.ptr, dw.vc.ptr, dw.bt.ptr,
                                dw.ctx.ptr, w.scale, sh["num_seqs"], sh["num_heads"],
                                sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
                                sh["max_num_blocks_per_seq"], 64, None)
    synchronize()
    assert L.swiftllm_hip_last_error() == 0
    assert_attention_close(dw.out.numpy(), _ref(w), "launch_paged_attention_v2")
    # an unsupported head_dim is refused without touching the output
    L.launch_paged_attention_v1(dw.out.ptr, dw.q.ptr, dw.kc.ptr, dw.vc.ptr, dw.bt.ptr, dw.ctx.ptr,
                                w.scale, sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], 96,
                                sh["block_size"], sh["max_num_blocks_per_seq"], None)
    assert L.swiftllm_hip_last_error() == pa.NotSupported.code


def test_paged_attention_op(dev):
    """PagedAttention.decode (paged_attention.rs:205-238): store the new K/V,
    then attend, from host-side tables."""
    rng = np.random.default_rng(41)
    cfg = pa.PagedAttentionConfig.new(32, 8, 128, 16)
    S, NB = 6, 64
    ctx = np.array([1, 16, 17, 100, 250, 33])
    perm = rng.permutation(NB)
    tables, pos = [], 0
    for L in ctx:
        n = (L + 15) // 16
        tables.append([int(b) for b in perm[pos:pos + n]])
        pos += n
    slots = [t[(L - 1) // 16] * 16 + (L - 1) % 16 for t, L in zip(tables, ctx)]
    kc = rng.standard_normal((NB, 8, 128, 16)).astype(np.float16)
    vc = rng.standard_normal((NB, 8, 128, 16)).astype(np.float16)
    q = rng.standard_normal((S, 1, 32, 128)).astype(np.float16)
    k = rng.standard_normal((S, 1, 8, 128)).astype(np.float16)
    v = rng.standard_normal((S, 1, 8, 128)).astype(np.float16)
    op = pa.PagedAttention(cfg, partition_size=32)
    kc_d, vc_d = DeviceArray.from_numpy(kc), DeviceArray.from_numpy(vc)
    out = op.decode(DeviceArray.from_numpy(q), DeviceArray.from_numpy(k), DeviceArray.from_numpy(v),
                    kc_d, vc_d, tables, list(ctx), slots).numpy()
    oracle.reshape_and_cache(k[:, 0], v[:, 0], kc, vc, np.array(slots, np.int32))
    bt, ctx32 = pa.BatchedCacheMetadata(), None
    for t, L in zip(tables, ctx):
        bt.add_sequence(pa.SequenceCacheMetadata(int(L), t), [])
    bt_arr, ctx32 = bt.pack(16)
    ref = oracle.decode_f64(q[:, 0], kc, vc, bt_arr, ctx32, cfg.scale)
    assert_attention_close(out[:, 0], ref, "PagedAttention.decode")
    with pytest.raises(pa.InvalidParameter):
        op.reshape_and_cache(DeviceArray.from_numpy(k), DeviceArray.from_numpy(v), kc_d, vc_d, slots[:-1])


def test_pool_past_two_gigaelements(dev):
    """A pool of 140,000 blocks (4.6 GB per cache at Hkv 8, D 128): element
    offsets pass 2^31, where the reference's int arithmetic (cu:86) wraps.
    Block tables point at the highest blocks; the K/V get there through
    reshape_and_cache on the device, and the decode must match the oracle on
    a compact relabelled copy of the same blocks, for every entry point."""
    S, H, Hkv, D, NB = 4, 32, 8, 128, 140_000
    ctx = np.array([1, 40, 129, 300], np.int32)
    nblk = (ctx + 15) // 16
    MB = int(nblk.max())
    rng = np.random.default_rng(41)
    high = NB - 1 - rng.permutation(2000)[: int(nblk.sum())]     # ids 138,000 .. 139,999
    bt = np.zeros((S, MB), np.int32)
    slots, keys, vals, pos = [], [], [], 0
    for s in range(S):
        bt[s, : nblk[s]] = high[pos: pos + nblk[s]]
        pos += nblk[s]
        for p in range(ctx[s]):
            slots.append(int(bt[s, p // 16]) * 16 + p % 16)
    T = len(slots)
    key = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    value = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    kc, vc = DeviceArray((NB, Hkv, D, 16), np.float16), DeviceArray((NB, Hkv, D, 16), np.float16)
    assert kc.nbytes > 2 ** 32
    pa.launch_reshape_and_cache(DeviceArray.from_numpy(key), DeviceArray.from_numpy(value), kc, vc,
                                DeviceArray.from_numpy(np.array(slots, np.int32)), T, Hkv, D, 16,
                                num_blocks=NB)
    # compact host copy: the used blocks relabelled 0..n-1
    used = np.unique(bt[bt > 0]) if (bt > 0).any() else np.array([], np.int64)
    relabel = {int(b): i for i, b in enumerate(used)}
    kc_h = np.zeros((len(used), Hkv, D, 16), np.float16)
    vc_h = np.zeros_like(kc_h)
    sl = np.array(slots)
    rb = np.array([relabel[int(x)] for x in sl // 16])
    kc_h[rb, :, :, sl % 16] = key
    vc_h[rb, :, :, sl % 16] = value
    bt_h = np.vectorize(lambda b: relabel.get(int(b), 0))(bt).astype(np.int32)
    q = rng.standard_normal((S, H, D)).astype(np.float16)
    scale = 1.0 / np.sqrt(D)
    ref = oracle.decode_f64(q, kc_h, vc_h, bt_h, ctx, scale)
    qd, btd, cd = DeviceArray.from_numpy(q), DeviceArray.from_numpy(bt), DeviceArray.from_numpy(ctx)
    out = DeviceArray((S, H, D), np.float16)
    pa.paged_attention_v1(out, qd, kc, vc, btd, cd, scale, S, H, Hkv, D, 16, MB, num_blocks=NB)
    synchronize()
    assert_attention_close(out.numpy(), ref, "v1 on a 140k-block pool")
    for ps in (32, 0):
        ws = pa.workspace(pa.paged_attention_v2_workspace_size(S, H, Hkv, D, 16, MB, ps))
        pa.paged_attention_v2(out, ws, qd, kc, vc, btd, cd, scale, S, H, Hkv, D, 16, MB, ps,
                              num_blocks=NB)
        synchronize()
        assert_attention_close(out.numpy(), ref, f"v2 ps={ps} on a 140k-block pool")
    kc.free()
    vc.free()


def _random_batch(rng, lens, H, Hkv, D, std=1.0, extra_blocks=4):
    """A decode workload with the given context lengths over a permuted pool."""
    lens = np.asarray(lens, np.int32)
    need = (np.maximum(lens, 0) + 15) // 16
    MB = max(int(need.max()), 1)
    NB = int(need.sum()) + extra_blocks
    perm = rng.permutation(NB).astype(np.int32)
    bt = np.zeros((len(lens), MB), np.int32)
    pos = 0
    for s, n in enumerate(need):
        bt[s, :n] = perm[pos:pos + n]
        pos += n
    kc = (rng.standard_normal((NB, Hkv, D, 16)) * std).astype(np.float16)
    vc = (rng.standard_normal((NB, Hkv, D, 16)) * std).astype(np.float16)
    q = (rng.standard_normal((len(lens), H, D)) * std).astype(np.float16)
    return workloads.DecodeWorkload("batch", q, kc, vc, bt, lens, 1.0 / np.sqrt(D))


@pytest.mark.parametrize("G", [8, 1])
def test_one_long_sequence_many_fragments(dev, G):
    """One 32768-token sequence (plus a short one) in balanced mode: the
    sequence spans hundreds of teams, so its reduce combines more than 64
    fragments per item (several passes of the one-wave combine); the
    partitioned modes combine 64 and 8 partitions (workgroup reduce)."""
    rng = np.random.default_rng(70 + G)
    w = _random_batch(rng, [32768, 37], H=8 * G, Hkv=8, D=128)
    dw = DeviceWorkload(w)
    ref = _ref(w)
    for ps in (0, 512, 4096):
        assert_attention_close(dw.run("v2", partition_size=ps), ref, f"long G={G} ps={ps}")


@pytest.fixture(scope="module")
def context_128k(dev):
    """One sequence of 131,077 tokens (Llama-3's 128k context plus a partial
    block) beside sequences of 3 and 700, at the 70B head layout (64 query
    heads, 8 kv heads): 8,244 blocks, 540 MB of K/V. NaN fills the slots
    past each context in its last block."""
    rng = np.random.default_rng(128)
    w = _random_batch(rng, [131_077, 3, 700], H=64, Hkv=8, D=128, extra_blocks=1)
    for s, L in enumerate(w.context_lens):
        j = (int(L) - 1) // 16
        valid = int(L) - 16 * j
        w.key_cache[w.block_tables[s, j], :, :, valid:] = np.nan
        w.value_cache[w.block_tables[s, j], :, :, valid:] = np.nan
    return DeviceWorkload(w), _ref(w)


@pytest.mark.parametrize("variant,ps", [("v1", None), ("v2", 512), ("v2", 16), ("v2", 0)])
def test_context_past_128k(context_128k, variant, ps):
    """The single pass over 8,193 blocks; split-K with 257 partitions of 512
    tokens and with 8,193 of 16 (the workgroup reduce's chunked loop many
    times over, and an 818 MB workspace); balanced mode."""
    dw, ref = context_128k
    assert_attention_close(dw.run(variant, partition_size=ps), ref, f"128k {variant} ps={ps}")


def test_more_sequences_than_the_lds_tables(dev):
    """4500 short sequences: the single pass drops its longest-first ranking
    (more than 128 sequences), the partition kernel takes one item per
    workgroup over the full grid (more than 4096), and balanced mode falls
    back to 512-token partitions (more than 4096)."""
    rng = np.random.default_rng(45)
    lens = rng.integers(0, 48, size=4500)
    w = _random_batch(rng, lens, H=4, Hkv=2, D=64)
    dw = DeviceWorkload(w)
    ref = _ref(w)
    live = lens > 0
    for variant, ps in (("v1", None), ("v2", 32), ("v2", 0)):
        out = dw.run(variant, partition_size=ps)
        assert np.all(out[~live] == 0), f"{variant} ps={ps}: empty sequences must be zero"
        assert_attention_close(out[live], ref[live], f"4500 seqs {variant} ps={ps}")


@pytest.mark.parametrize("S,ps", [(300, 64), (1100, 32), (4096, 16)])
def test_partition_items_longest_first_cover_every_partition(dev, S, ps):
    """The split-K kernel orders its items longest first in a list that every
    workgroup builds in its own LDS; the items of one list position are run
    by different workgroups (one per kv head), so the list must come out the
    same in each. Ragged batches of more than one 256-sequence chunk, at
    partitions small enough that every workgroup walks many items and every
    length class holds ties, with empty sequences: every partition of every
    sequence is attended exactly once (a missing one leaves the output
    unwritten or the reduce short of a fragment)."""
    rng = np.random.default_rng(S + ps)
    lens = np.clip(np.rint(np.exp(rng.normal(np.log(90.0), 1.0, size=S))), 0, 1500).astype(np.int64)
    lens[rng.choice(S, size=S // 10, replace=False)] = 0
    w = _random_batch(rng, lens, H=8, Hkv=2, D=64)
    out = DeviceWorkload(w).run("v2", partition_size=ps)
    live = lens > 0
    assert np.all(out[~live] == 0), "empty sequences must be zero"
    assert_attention_close(out[live], _ref(w)[live], f"{S} ragged seqs ps={ps}")


@pytest.mark.parametrize("H,Hkv,D", [(64, 8, 128), (64, 2, 128), (48, 2, 128), (16, 1, 128), (32, 8, 64)])
def test_partition_streams_ragged(dev, H, Hkv, D):
    """Split-K over short partitions of a batch with few sequences runs as
    partition streams: equal block ranges per team of waves, cut at partition
    ends and at range boundaries. Ragged contexts with empty sequences put
    range boundaries inside partitions, at partition starts and at sequence
    starts; 16-token partitions make every block a partition, and the 2-kv-head
    layouts (G = 32, two head chunks; G = 24, the second chunk 8 heads wide)
    give small teams whose ranges are shorter than a partition; G = 16 with
    one kv head gives one-wave teams. Pieces that end inside a wave's range
    are held in LDS and written with the wave's last piece."""
    rng = np.random.default_rng(H + Hkv + D)
    S = 40
    lens = np.clip(np.rint(np.exp(rng.normal(np.log(1500.0), 1.2, size=S))), 1, 20000).astype(np.int64)
    lens[rng.choice(S, size=5, replace=False)] = 0
    w = _random_batch(rng, lens, H=H, Hkv=Hkv, D=D)
    dw = DeviceWorkload(w)
    ref = _ref(w)
    live = lens > 0
    for ps in (16, 256, 512, 1024):
        out = dw.run("v2", partition_size=ps)
        assert np.all(out[~live] == 0), f"ps={ps}: empty sequences must be zero"
        assert_attention_close(out[live], ref[live], f"streams H{H} Hkv{Hkv} D{D} ps={ps}")


@pytest.mark.parametrize("D", [128, 64])
def test_item_reduce_many_partitions(dev, D):
    """Split-K over the item kernel (80 sequences: more than a quarter of the
    teams a partition stream needs) with up to 188 partitions per sequence:
    above 16 partitions the reduce runs on four waves per head (16, 64), at
    most 16 on one wave (256); empty and one-block sequences included."""
    rng = np.random.default_rng(91 + D)
    S = 80
    lens = np.clip(np.rint(np.exp(rng.normal(np.log(700.0), 1.0, size=S))), 1, 3000).astype(np.int64)
    lens[:3] = [0, 1, 3000]
    w = _random_batch(rng, lens, H=32, Hkv=8, D=D)
    dw = DeviceWorkload(w)
    ref = _ref(w)
    live = lens > 0
    for ps in (16, 64, 256):
        out = dw.run("v2", partition_size=ps)
        assert np.all(out[~live] == 0), f"ps={ps}: empty sequences must be zero"
        assert_attention_close(out[live], ref[live], f"item reduce D{D} ps={ps}")


@pytest.mark.parametrize("D", [128, 64])
def test_partition_stream_reduce_fragment_counts(dev, D):
    """The reduce of a head with more than 16 fragments runs on four waves,
    each combining 16-fragment chunks, merged through LDS. With 16-token
    partitions every block is a partition and every range boundary falls on a
    partition start, so a sequence of n blocks leaves exactly n fragments per
    head. The counts cross a wave's chunk (16 / 17), one pass of the four
    waves (63 / 64 / 65) and several passes (129, 200), beside sequences of 1
    block (written directly), 2 and 8 blocks and an empty one; some last
    blocks are partial."""
    rng = np.random.default_rng(77 + D)
    blocks = np.array([1, 2, 8, 9, 16, 17, 63, 64, 65, 129, 200, 0])
    lens = blocks * 16 - (np.arange(len(blocks)) % 3) * 5
    lens[blocks == 0] = 0
    w = _random_batch(rng, lens, H=64, Hkv=8, D=D)
    out = DeviceWorkload(w).run("v2", partition_size=16)
    live = lens > 0
    assert np.all(out[~live] == 0), "empty sequences must be zero"
    assert_attention_close(out[live], _ref(w)[live], f"reduce fragment counts D{D}")
