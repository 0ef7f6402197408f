"""Paged prefill on the GPU against oracle.prefill_numpy (float64), to the
attention tolerance (max_abs <= 2e-3, max_rel <= 1e-2 with a 1e-3 floor):
packed prompts of ragged lengths around block edges, GQA groups from 1 to
32, head_dim 64 and 128, NaN in every unused cache slot, the bounded status
entry, the bindings twin and PagedAttention.prefill."""

import dataclasses

import numpy as np
import pytest

import oracle
from helpers import assert_attention_close
from swiftllm_amd import paged_attention as pa
from swiftllm_amd import workloads
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def _run(w, entry="status", max_len=None):
    T, H, D = w.q.shape
    Hkv = w.key_cache.shape[1]
    S = len(w.context_lens)
    max_len = int(w.context_lens.max()) if max_len is None else max_len
    out = DeviceArray((T, H, D), np.float16)
    out.fill_byte(0xFF)
    q = DeviceArray.from_numpy(w.q)
    kc, vc = DeviceArray.from_numpy(w.key_cache), DeviceArray.from_numpy(w.value_cache)
    sm, ctx = DeviceArray.from_numpy(w.slot_mapping), DeviceArray.from_numpy(w.context_lens)
    if entry == "status":
        pa.launch_paged_prefill(out, q, kc, vc, sm, ctx, w.scale, S, H, Hkv, D, 16, max_len,
                                num_blocks=w.key_cache.shape[0])
    else:
        pa.paged_attention_prefill(out, q, kc, vc, sm, ctx,
                                   pa.PagedAttentionParams(S, H, Hkv, D, 16, w.scale, max_len))
    synchronize()
    return out.numpy()


def _ref(w):
    return oracle.prefill_numpy(w.q, w.key_cache, w.value_cache, w.slot_mapping, w.context_lens,
                                w.scale)


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (8, 8, 64), (64, 8, 128), (16, 1, 64),
                                     (32, 1, 128), (12, 4, 64)])
def test_prefill_gqa_shapes(dev, H, Hkv, D):
    lens = (1, 15, 16, 17, 70, 129)
    w = workloads.prefill_config(lens, H, Hkv, D, seed=H * 10 + Hkv + D)
    assert_attention_close(_run(w), _ref(w), f"prefill H{H} Hkv{Hkv} D{D}")


@pytest.mark.parametrize("entry", ["status", "params"])
def test_prefill_long_prompts(dev, entry):
    """Llama-3-8B layer heads, two long prompts and a short one."""
    w = workloads.prefill_config((1024, 517, 3), 32, 8, 128, seed=7)
    assert_attention_close(_run(w, entry), _ref(w), f"prefill long {entry}")


@pytest.mark.parametrize("H,Hkv,D", [(32, 8, 128), (16, 4, 64)])
def test_prefill_walks_past_two_id_chunks(dev, H, Hkv, D):
    """Key walks of more than 128 blocks: the kernel keeps the block ids of
    its walk in chunks of 64 blocks, double-buffered, so a 2600-token prompt
    crosses into the second chunk and reuses the first chunk's buffer for the
    third; 1100 tokens end just past the first chunk; 5 is a one-block walk."""
    w = workloads.prefill_config((2600, 1100, 5), H, Hkv, D, seed=21 + D)
    assert_attention_close(_run(w), _ref(w), f"prefill id chunks H{H} Hkv{Hkv} D{D}")


@pytest.mark.parametrize("scale", [-0.0883883, 0.0, 0.3])
def test_prefill_scale_signs(dev, scale):
    """A positive scale takes the kernel's path with the scale folded into the
    exp2 argument (max on unscaled scores); zero and negative scales take the
    plain path (max on scaled scores). Both against the oracle."""
    w = dataclasses.replace(workloads.prefill_config((1, 17, 70, 129), 32, 8, 128, seed=11),
                            scale=scale)
    assert_attention_close(_run(w), _ref(w), f"prefill scale {scale}")


def test_prefill_key_cache_8_byte_aligned(dev):
    """A key cache that is 8- but not 16-byte aligned takes the kernel's
    register path for K (the default path copies K tiles into LDS with
    16-byte loads); both against the oracle."""
    w = workloads.prefill_config((1, 17, 70, 129), 32, 8, 128, seed=13)
    T, H, D = w.q.shape
    S = len(w.context_lens)
    kc_buf = DeviceArray((w.key_cache.nbytes + 16,), np.uint8)
    kc_bytes = np.zeros(w.key_cache.nbytes + 16, np.uint8)
    kc_bytes[8:8 + w.key_cache.nbytes] = w.key_cache.view(np.uint8).ravel()
    kc_buf.upload(kc_bytes)
    out = DeviceArray((T, H, D), np.float16)
    q = DeviceArray.from_numpy(w.q)
    vc = DeviceArray.from_numpy(w.value_cache)
    sm, ctx = DeviceArray.from_numpy(w.slot_mapping), DeviceArray.from_numpy(w.context_lens)
    pa.launch_paged_prefill(out, q, kc_buf.ptr + 8, vc, sm, ctx, w.scale, S, H, 8, D, 16,
                            int(w.context_lens.max()), num_blocks=w.key_cache.shape[0])
    synchronize()
    assert_attention_close(out.numpy(), _ref(w), "prefill, key cache at +8 bytes")


def test_prefill_empty_and_zero_length_sequences(dev):
    w = workloads.prefill_config((0, 33, 0, 5), 8, 2, 64, seed=8)
    out = _run(w)
    assert_attention_close(out, _ref(w), "prefill with empty prompts")


def test_prefill_grid_rounds_past_65535(dev):
    """65535 one-token prompts with 16 kv heads: 1,048,560 (sequence, kv head)
    units, so the launch needs 131,070 rounds of 8 units, more than one grid
    row (65535) holds, and the second grid plane runs. A one-token prompt
    attends only to itself: out = its own V (the prompts share a pool of 64
    blocks; slots 1..15 of every block hold NaN)."""
    S, H, Hkv, D, NB = 65535, 16, 16, 64, 64
    rng = np.random.default_rng(5)
    q = (rng.standard_normal((S, H, D)) * 0.5).astype(np.float16)
    kc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    vc = np.full((NB, Hkv, D, 16), np.nan, np.float16)
    kc[:, :, :, 0] = (rng.standard_normal((NB, Hkv, D)) * 0.5).astype(np.float16)
    vc[:, :, :, 0] = (rng.standard_normal((NB, Hkv, D)) * 0.5).astype(np.float16)
    block = np.arange(S, dtype=np.int32) % NB
    slots = (block * 16).astype(np.int32)
    ctx = np.ones(S, np.int32)
    out = DeviceArray((S, H, D), np.float16)
    out.fill_byte(0xFF)
    pa.launch_paged_prefill(out, DeviceArray.from_numpy(q), DeviceArray.from_numpy(kc),
                            DeviceArray.from_numpy(vc), DeviceArray.from_numpy(slots),
                            DeviceArray.from_numpy(ctx), 1.0 / 8.0, S, H, Hkv, D, 16, 1,
                            num_blocks=NB)
    synchronize()
    expect = vc[block, :, :, 0]  # [S, Hkv, D]; G = 1: head h reads kv head h
    assert_attention_close(out.numpy(), expect, "prefill 65535 one-token prompts")


def test_prefill_max_len_above_every_prompt(dev):
    """A generous max_context_len only adds workgroups that exit at once."""
    w = workloads.prefill_config((20, 50), 8, 2, 64, seed=9)
    assert_attention_close(_run(w, max_len=4096), _ref(w), "prefill max_len 4096")


def test_prefill_out_of_pool_blocks_are_skipped(dev):
    """With the pool bound, a prompt whose slots point past the pool reads
    nothing out of bounds; its outputs stay finite and the others are exact."""
    w = workloads.prefill_config((40, 24), 8, 2, 64, seed=10)
    NB = w.key_cache.shape[0]
    w.slot_mapping[40:] = (NB + 3) * 16 + np.arange(24) % 16   # second prompt: outside the pool
    out = _run(w)
    ref = _ref_first(w, 40)
    assert_attention_close(out[:40], ref, "prefill in-pool prompt")
    assert np.all(np.isfinite(out[40:].astype(np.float64)))


@pytest.mark.parametrize("key_offset", [0, 8])
def test_prefill_padding_slots_attend_nothing(dev, key_offset):
    """A prompt whose slots are -1 (padding, as reshape_and_cache skips them)
    reads no block: -1 // 16 must not become block 0. Its rows attend to no
    key and come out as zeros; the prompts beside it are exact. key_offset 8
    runs the register path for K, 0 the LDS path."""
    w = workloads.prefill_config((40, 24, 19), 8, 2, 64, seed=12)
    w.slot_mapping[40:64] = -1
    T, H, D = w.q.shape
    S = len(w.context_lens)
    kc_buf = DeviceArray((w.key_cache.nbytes + 16,), np.uint8)
    kc_bytes = np.zeros(w.key_cache.nbytes + 16, np.uint8)
    kc_bytes[key_offset:key_offset + w.key_cache.nbytes] = w.key_cache.view(np.uint8).ravel()
    kc_buf.upload(kc_bytes)
    out = DeviceArray((T, H, D), np.float16)
    out.fill_byte(0xFF)
    sm, ctx = DeviceArray.from_numpy(w.slot_mapping), DeviceArray.from_numpy(w.context_lens)
    pa.launch_paged_prefill(out, DeviceArray.from_numpy(w.q), kc_buf.ptr + key_offset,
                            DeviceArray.from_numpy(w.value_cache), sm, ctx, w.scale, S, H, 2, D, 16,
                            int(w.context_lens.max()), num_blocks=w.key_cache.shape[0])
    synchronize()
    got = out.numpy()
    assert np.array_equal(got[40:64].view(np.uint16), np.zeros((24, H, D), np.uint16))
    ref_a = oracle.prefill_numpy(w.q[:40], w.key_cache, w.value_cache, w.slot_mapping[:40],
                                 w.context_lens[:1], w.scale)
    ref_c = oracle.prefill_numpy(w.q[64:], w.key_cache, w.value_cache, w.slot_mapping[64:],
                                 w.context_lens[2:], w.scale)
    assert_attention_close(got[:40], ref_a, "prefill prompt before the padding")
    assert_attention_close(got[64:], ref_c, "prefill prompt after the padding")


def _ref_first(w, n):
    return oracle.prefill_numpy(w.q[:n], w.key_cache, w.value_cache, w.slot_mapping[:n],
                                w.context_lens[:1], w.scale)


def test_paged_attention_prefill_op(dev):
    """PagedAttention.prefill (paged_attention.rs:154-189): stores K/V through
    slot_mapping, then the causal attention; query [B, S, H, D]."""
    B, S, H, Hkv, D = 3, 37, 8, 2, 64
    w = workloads.prefill_config((S,) * B, H, Hkv, D, seed=11, poison=True)
    kc0 = np.full_like(w.key_cache, np.nan)
    vc0 = np.full_like(w.value_cache, np.nan)
    op = pa.PagedAttention(pa.PagedAttentionConfig.new(H, Hkv, D, 16))
    kc, vc = DeviceArray.from_numpy(kc0), DeviceArray.from_numpy(vc0)
    out = op.prefill(DeviceArray.from_numpy(w.q.reshape(B, S, H, D)),
                     DeviceArray.from_numpy(w.key.reshape(B, S, Hkv, D)),
                     DeviceArray.from_numpy(w.value.reshape(B, S, Hkv, D)),
                     kc, vc, list(w.slot_mapping))
    assert out.shape == (B, S, H, D)
    assert_attention_close(out.numpy().reshape(B * S, H, D), _ref(w), "PagedAttention.prefill")
    b, o = w.slot_mapping // 16, w.slot_mapping % 16
    assert np.array_equal(kc.numpy()[b, :, :, o].view(np.uint16), w.key.view(np.uint16))
