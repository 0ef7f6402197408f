"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from computations independent of oracle/):
the oracle must reproduce them on the CPU, and the library through the C ABI
on the GPU. Decode is held to the attention tolerance, everything else is
bit-exact (MoE weights within 1e-6 on the GPU)."""

from pathlib import Path

import numpy as np
import pytest

import oracle
from helpers import DeviceWorkload, assert_attention_close
from swiftllm_amd import moe, workloads
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, synchronize

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _decode_cases():
    z = _load("decode_small.npz")
    names = sorted({k.split("_", 1)[0] for k in z})
    return {c: {k.split("_", 1)[1]: v for k, v in z.items() if k.startswith(c + "_")} for c in names}


DECODE = _decode_cases()


def _workload(case):
    return workloads.DecodeWorkload(
        name="golden", q=case["q"], key_cache=case["key_cache"], value_cache=case["value_cache"],
        block_tables=case["block_tables"], context_lens=case["context_lens"],
        scale=float(case["scale"]), partition_size=16)


# --------------------------------------------------------------------------- CPU
@pytest.mark.parametrize("name", sorted(DECODE))
def test_oracle_decode_matches_golden(name):
    c = DECODE[name]
    for fn in (oracle.decode_f64, oracle.decode_numpy):
        out = fn(c["q"], c["key_cache"], c["value_cache"], c["block_tables"], c["context_lens"],
                 float(c["scale"]))
        assert np.abs(out - c["expected"]).max() < 1e-12, fn.__name__


def test_oracle_cache_matches_golden():
    z = _load("cache_small.npz")
    for fn in (oracle.reshape_and_cache, oracle.reshape_and_cache_numpy):
        kc, vc = z["key_cache_in"].copy(), z["value_cache_in"].copy()
        fn(z["key"], z["value"], kc, vc, z["slot_mapping"])
        assert np.array_equal(kc.view(np.uint16), z["key_cache_expected"].view(np.uint16))
        assert np.array_equal(vc.view(np.uint16), z["value_cache_expected"].view(np.uint16))


def test_oracle_moe_matches_golden():
    z = _load("moe_small.npz")
    ids, w = oracle.moe_route(z["logits"], int(z["top_k"]))
    assert np.array_equal(ids, z["expert_ids"])
    assert np.abs(w - z["weights"]).max() < 1e-15
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, z["logits"].shape[1])
    assert np.array_equal(counts, z["counts"])
    assert np.array_equal(offsets, z["offsets"])
    assert np.array_equal(inverse, z["inverse"])
    assert np.array_equal(sorted_ids, z["sorted_token_ids"])


# --------------------------------------------------------------------------- GPU
@pytest.mark.gpu
@pytest.mark.parametrize("name", sorted(DECODE))
@pytest.mark.parametrize("variant,ps", [("v1", None), ("v2", 16), ("v2", 0), ("decode", None)])
def test_gpu_decode_matches_golden(dev, name, variant, ps):
    c = DECODE[name]
    out = DeviceWorkload(_workload(c)).run(variant, partition_size=ps)
    assert_attention_close(out, c["expected"], f"golden {name} {variant} ps={ps}")


@pytest.mark.gpu
def test_gpu_cache_matches_golden(dev):
    z = _load("cache_small.npz")
    T, Hkv, D = z["key"].shape
    NB = z["key_cache_in"].shape[0]
    kc = DeviceArray.from_numpy(z["key_cache_in"])
    vc = DeviceArray.from_numpy(z["value_cache_in"])
    pa.launch_reshape_and_cache(DeviceArray.from_numpy(z["key"]), DeviceArray.from_numpy(z["value"]),
                                kc, vc, DeviceArray.from_numpy(z["slot_mapping"]), T, Hkv, D, 16,
                                num_blocks=NB)
    synchronize()
    assert np.array_equal(kc.numpy().view(np.uint16), z["key_cache_expected"].view(np.uint16))
    assert np.array_equal(vc.numpy().view(np.uint16), z["value_cache_expected"].view(np.uint16))


@pytest.mark.gpu
@pytest.mark.parametrize("fused", [False, True])
def test_gpu_moe_matches_golden(dev, fused):
    z = _load("moe_small.npz")
    T, E = z["logits"].shape
    K, hidden = int(z["top_k"]), z["x"].shape[1]
    logits, x = DeviceArray.from_numpy(z["logits"]), DeviceArray.from_numpy(z["x"])
    ids, w = DeviceArray((T, K), np.int32), DeviceArray((T, K), np.float32)
    bufs = moe.DispatchBuffers.allocate(T, E, K, hidden)
    if fused:
        moe.moe_route_dispatch(logits, x, K, ids, w, bufs)
    else:
        moe.moe_route(logits, K, ids, w)
        moe.moe_dispatch(ids, x, E, bufs)
    synchronize()
    assert np.array_equal(ids.numpy(), z["expert_ids"])
    assert np.abs(w.numpy() - z["weights"]).max() <= 1e-6
    assert np.array_equal(bufs.counts.numpy(), z["counts"])
    assert np.array_equal(bufs.offsets.numpy(), z["offsets"])
    assert np.array_equal(bufs.inverse.numpy(), z["inverse"])
    assert np.array_equal(bufs.sorted_token_ids.numpy(), z["sorted_token_ids"])
    assert np.array_equal(bufs.x_perm.numpy().view(np.uint16), z["x_perm"].view(np.uint16))
