"""reshape_and_cache on the GPU: bit-exact over the whole pool against the C
oracle (cu:167-199); untouched slots keep their sentinel."""

import numpy as np
import pytest

import oracle
from swiftllm_amd import _lib
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu

SENTINEL = 0x7E00  # an fp16 NaN pattern nobody writes


def _case(rng, T, Hkv, D, BS, NB, neg=0):
    slots = rng.choice(NB * BS, size=T, replace=False).astype(np.int32)
    if neg:
        slots[rng.choice(T, size=neg, replace=False)] = -1
    key = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    value = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    kc = np.full((NB, Hkv, D, BS), SENTINEL, np.uint16).view(np.float16)
    vc = np.full((NB, Hkv, D, BS), SENTINEL, np.uint16).view(np.float16)
    return key, value, kc, vc, slots


def _run(key, value, kc, vc, slots, entry):
    T, Hkv, D = key.shape
    NB, _, _, BS = kc.shape
    k_d, v_d = DeviceArray.from_numpy(key), DeviceArray.from_numpy(value)
    kc_d, vc_d = DeviceArray.from_numpy(kc), DeviceArray.from_numpy(vc)
    s_d = DeviceArray.from_numpy(slots)
    if entry == "status":
        pa.launch_reshape_and_cache(k_d, v_d, kc_d, vc_d, s_d, T, Hkv, D, BS, num_blocks=NB)
    elif entry == "params":
        pa.reshape_and_cache(k_d, v_d, kc_d, vc_d, s_d, pa.ReshapeCacheParams(T, Hkv, D, BS))
    elif entry == "dropin":
        _lib.lib().launch_reshape_and_cache(k_d.ptr, v_d.ptr, kc_d.ptr, vc_d.ptr, s_d.ptr, T, Hkv, D,
                                            BS, None)
        assert _lib.lib().swiftllm_hip_last_error() == 0
    synchronize()
    return kc_d.numpy(), vc_d.numpy()


@pytest.mark.parametrize("entry", ["status", "params", "dropin"])
@pytest.mark.parametrize("T,Hkv,D,BS,NB,neg", [
    (4, 8, 64, 16, 128, 0),        # config-1 shapes
    (256, 8, 128, 16, 2000, 0),    # config-4 shapes (one token per sequence)
    (300, 8, 128, 16, 400, 17),    # padding tokens (slot -1) are skipped
    (64, 2, 80, 8, 50, 0),         # other head_dim / block_size
    (33, 1, 256, 32, 10, 3),
])
def test_reshape_and_cache_bit_exact(dev, entry, T, Hkv, D, BS, NB, neg):
    rng = np.random.default_rng(T * 7 + D)
    key, value, kc, vc, slots = _case(rng, T, Hkv, D, BS, NB, neg)
    gk, gv = _run(key, value, kc, vc, slots, entry)
    rk, rv = kc.copy(), vc.copy()
    oracle.reshape_and_cache(key, value, rk, rv, slots)
    assert np.array_equal(gk.view(np.uint16), rk.view(np.uint16))
    assert np.array_equal(gv.view(np.uint16), rv.view(np.uint16))


def test_prefill_run_of_slots(dev):
    """Consecutive slots of one sequence (prefill) fill whole blocks and cross
    block boundaries."""
    rng = np.random.default_rng(5)
    T, Hkv, D, BS, NB = 70, 8, 128, 16, 20
    table = rng.permutation(NB)[:5]
    slots = np.array(oracle.slot_mapping(list(table), BS, 3, T), np.int32)
    key = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    value = rng.standard_normal((T, Hkv, D)).astype(np.float16)
    kc = np.full((NB, Hkv, D, BS), SENTINEL, np.uint16).view(np.float16)
    vc = kc.copy()
    gk, gv = _run(key, value, kc, vc, slots, "status")
    rk, rv = kc.copy(), vc.copy()
    oracle.reshape_and_cache_numpy(key, value, rk, rv, slots)
    assert np.array_equal(gk.view(np.uint16), rk.view(np.uint16))
    assert np.array_equal(gv.view(np.uint16), rv.view(np.uint16))


def test_out_of_pool_slots_skipped(dev):
    rng = np.random.default_rng(9)
    key, value, kc, vc, slots = _case(rng, 40, 4, 64, 16, 30)
    slots[::5] = 30 * 16 + 7  # past the pool
    gk, gv = _run(key, value, kc, vc, slots, "status")
    keep = np.where(slots < 30 * 16, slots, -1).astype(np.int32)
    rk, rv = kc.copy(), vc.copy()
    oracle.reshape_and_cache(key, value, rk, rv, keep)
    assert np.array_equal(gk.view(np.uint16), rk.view(np.uint16))
