"""Known-answer tests from the reference's own unit tests, applied to the
host-side mirror (swiftllm_amd.paged_attention) and the oracle. Paths are
relative to the reference repository."""

import math

import numpy as np
import pytest

import oracle
from swiftllm_amd import paged_attention as pa


def test_kv_cache_config_sizes():
    """crates/swiftllm-core/src/memory/kv_cache.rs:304-320."""
    cfg = pa.KvCacheConfig(num_layers=32, num_kv_heads=8, head_dim=128, block_size=16, dtype="float16")
    assert cfg.token_size_bytes() == 4096
    assert cfg.block_size_bytes() == 65536
    # and the device layout holds exactly that: K and V tiles of one block
    assert 2 * (8 * 128 * 16) * 2 == cfg.block_size_bytes()


def test_paged_attention_config():
    """crates/swiftllm-core/src/memory/paged_attention.rs:412-420."""
    cfg = pa.PagedAttentionConfig.new(32, 8, 128, 16)
    assert cfg.num_heads == 32
    assert cfg.num_kv_heads == 8
    assert cfg.num_query_groups() == 4
    assert abs(cfg.scale - 1.0 / math.sqrt(128.0)) < 1e-6


def test_blocks_needed():
    """crates/swiftllm-core/src/memory/block_manager.rs:595-617: 100 tokens -> 7 blocks."""
    assert pa.blocks_needed(100, 16) == 7
    assert oracle.blocks_needed(100, 16) == 7
    assert pa.blocks_needed(0, 16) == 0 and pa.blocks_needed(16, 16) == 1 and pa.blocks_needed(17, 16) == 2


def test_batched_cache_metadata():
    """crates/swiftllm-core/src/memory/kv_cache.rs:337-360."""
    batch = pa.BatchedCacheMetadata()
    batch.add_sequence(pa.SequenceCacheMetadata(100, [0, 1, 2, 3, 4, 5, 6]), [0, 1, 2])
    batch.add_sequence(pa.SequenceCacheMetadata(50, [7, 8, 9, 10]), [3, 4])
    assert batch.batch_size() == 2
    assert batch.max_context_len == 100
    assert batch.context_lens == [100, 50]
    assert len(batch.slot_mapping) == 5
    bt, ctx = batch.pack(16)
    assert bt.shape == (2, 7)
    assert bt[0].tolist() == [0, 1, 2, 3, 4, 5, 6]
    assert bt[1].tolist() == [7, 8, 9, 10, 0, 0, 0]
    assert ctx.tolist() == [100, 50]


def test_decode_input_max_context_len():
    """crates/swiftllm-core/src/memory/paged_attention.rs:446-463."""
    batch = pa.BatchedCacheMetadata()
    batch.add_sequence(pa.SequenceCacheMetadata(100, [0, 1, 2, 3, 4, 5, 6]), [100])
    batch.add_sequence(pa.SequenceCacheMetadata(90, [7, 8, 9, 10, 11, 12]), [200])
    assert batch.max_context_len == 100
    assert batch.slot_mapping == [100, 200]


def test_sequence_cache_metadata():
    """crates/swiftllm-core/src/memory/kv_cache.rs:322-335."""
    m = pa.SequenceCacheMetadata()
    assert m.cache_len == 0 and m.num_blocks() == 0
    m.block_table += [0, 5]
    m.cache_len = 32
    assert m.num_blocks() == 2


def test_data_type_sizes():
    """crates/swiftllm-core/src/config.rs:638-643."""
    assert pa._DTYPE_BYTES["float32"] == 4
    assert pa._DTYPE_BYTES["float16"] == 2
    assert pa._DTYPE_BYTES["int8"] == 1


def test_attention_config_head_dim_and_gqa():
    """crates/swiftllm-models/src/layers/attention.rs:359-365: hidden 4096 over
    32 heads gives head_dim 128, and 8 kv heads make it GQA."""
    cfg = pa.PagedAttentionConfig.new(32, 8, 4096 // 32, 16)
    assert cfg.head_dim == 128
    assert cfg.num_query_groups() > 1


@pytest.mark.parametrize("table,start,n", [([3, 7], 14, 5), ([0], 0, 16), ([9, 2, 5], 31, 17), ([4], 3, 0)])
def test_slot_mapping_closed_form(table, start, n):
    """kv_cache.rs:199-212: slot = table[pos / bs] * bs + pos % bs."""
    got = pa.get_slot_mapping(table, 16, start, n)
    want = [table[p // 16] * 16 + p % 16 for p in range(start, start + n)]
    assert got.tolist() == want
    assert oracle.slot_mapping(table, 16, start, n) == want


def test_slot_mapping_known_values():
    assert pa.get_slot_mapping([3, 7], 16, 14, 5).tolist() == [62, 63, 112, 113, 114]


def test_slot_mapping_unallocated_block():
    """kv_cache.rs:203-208: a position past the table is an error."""
    with pytest.raises(pa.InvalidParameter, match="not allocated"):
        pa.get_slot_mapping([3, 7], 16, 30, 3)
    with pytest.raises(KeyError):
        oracle.slot_mapping([3, 7], 16, 30, 3)


def test_slot_mapping_int32_narrowing():
    """Slots are narrowed to int32 at the ABI (bindings.rs:100); a slot that
    does not fit is refused instead of wrapping."""
    with pytest.raises(pa.InvalidParameter, match="int32"):
        pa.get_slot_mapping([2**28], 16, 0, 1)


def test_pack_block_tables_errors():
    batch = pa.BatchedCacheMetadata()
    batch.add_sequence(pa.SequenceCacheMetadata(40, [1, 2]), [])  # needs 3 blocks, has 2
    with pytest.raises(pa.InvalidParameter, match="needs 3 blocks"):
        batch.pack(16)
    batch = pa.BatchedCacheMetadata()
    batch.add_sequence(pa.SequenceCacheMetadata(40, [1, 2, 3]), [])
    with pytest.raises(pa.InvalidParameter):
        batch.pack(16, max_blocks_per_seq=2)


def test_pack_block_tables_null_block_ids():
    """A null block_ids with a non-empty table is refused, not dereferenced;
    with every table empty it is accepted (nothing is read)."""
    from swiftllm_amd import _lib

    L = _lib.lib()
    offs = np.array([0, 2], np.uint64)
    ctx = np.array([20], np.uint64)
    bt = np.zeros((1, 4), np.int32)
    cl = np.zeros(1, np.int32)
    rc = L.swiftllm_hip_pack_block_tables(None, offs.ctypes.data, ctx.ctypes.data, 1, 16, 4,
                                          bt.ctypes.data, cl.ctypes.data)
    assert rc == pa.InvalidParameter.code
    assert "block_ids" in _lib.last_error()[1]
    offs0 = np.array([0, 0], np.uint64)
    ctx0 = np.array([0], np.uint64)
    rc = L.swiftllm_hip_pack_block_tables(None, offs0.ctypes.data, ctx0.ctypes.data, 1, 16, 4,
                                          bt.ctypes.data, cl.ctypes.data)
    assert rc == 0 and cl[0] == 0 and not bt.any()


def test_pack_block_tables_random():
    rng = np.random.default_rng(0)
    batch = pa.BatchedCacheMetadata()
    tables, lens = [], []
    for _ in range(20):
        L = int(rng.integers(0, 300))
        n = oracle.blocks_needed(L, 16) + int(rng.integers(0, 3))
        t = [int(x) for x in rng.integers(0, 10_000, n)]
        tables.append(t)
        lens.append(L)
        batch.add_sequence(pa.SequenceCacheMetadata(L, t), [])
    bt, ctx = batch.pack(16)
    assert ctx.tolist() == lens
    for s, t in enumerate(tables):
        assert bt[s, :len(t)].tolist() == t
        assert np.all(bt[s, len(t):] == 0)


def test_paged_attention_op_rejects_unimplemented_options():
    """Sliding window and ALiBi are declared (paged_attention.rs:39-43, 67-77)
    but no kernel of the reference implements them."""
    op = pa.PagedAttention(pa.PagedAttentionConfig.new(32, 8, 128, 16).with_alibi())
    with pytest.raises(pa.NotSupported):
        op._validate()
    op = pa.PagedAttention(pa.PagedAttentionConfig.new(32, 8, 128, 16).with_sliding_window(4096))
    with pytest.raises(pa.NotSupported):
        op._validate()
