"""MoE routing and dispatch on the GPU: expert ids, counts, offsets, inverse
index, sorted token ids and permuted rows bit-exact against the oracle;
routing weights within 1e-6 of the fp64 oracle."""

import numpy as np
import pytest

import oracle
from swiftllm_amd import moe, workloads
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


def _route(logits, K):
    T, E = logits.shape
    ids = DeviceArray((T, K), np.int32)
    w = DeviceArray((T, K), np.float32)
    moe.moe_route(DeviceArray.from_numpy(logits), K, ids, w)
    synchronize()
    return ids.numpy(), w.numpy()


def _dispatch(ids, x, E, with_rows=True):
    T, K = ids.shape
    hidden = x.shape[1]
    bufs = moe.DispatchBuffers.allocate(T, E, K, hidden, with_rows=with_rows)
    moe.moe_dispatch(DeviceArray.from_numpy(ids), DeviceArray.from_numpy(x), E, bufs)
    synchronize()
    return bufs


def _route_dispatch(logits, x, K, with_rows=True):
    """The fused entry point, on a workspace filled with 0xFF bytes."""
    T, E = logits.shape
    ids = DeviceArray((T, K), np.int32)
    w = DeviceArray((T, K), np.float32)
    bufs = moe.DispatchBuffers.allocate(T, E, K, x.shape[1], with_rows=with_rows)
    bufs.workspace.fill_byte(0xFF)
    moe.moe_route_dispatch(DeviceArray.from_numpy(logits), DeviceArray.from_numpy(x), K, ids, w,
                           bufs)
    synchronize()
    return ids.numpy(), w.numpy(), bufs


def _check_dispatch(ids, x, E, bufs, with_rows=True):
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, E)
    assert np.array_equal(bufs.counts.numpy(), counts)
    assert np.array_equal(bufs.offsets.numpy(), offsets)
    assert np.array_equal(bufs.inverse.numpy(), inverse)
    n = int(offsets[-1])
    assert np.array_equal(bufs.sorted_token_ids.numpy()[:n], sorted_ids)
    if with_rows:
        xp = bufs.x_perm.numpy()
        assert np.array_equal(xp[:n].view(np.uint16), x[sorted_ids].view(np.uint16))


def test_config5_mixtral(dev):
    wl = workloads.moe_config(seed=5)
    ids, w = _route(wl.logits, wl.top_k)
    rids, rw = oracle.moe_route(wl.logits, wl.top_k)
    assert np.array_equal(ids, rids)
    assert np.abs(w - rw).max() <= 1e-6
    bufs = _dispatch(ids, wl.x, wl.num_experts)
    _check_dispatch(ids, wl.x, wl.num_experts, bufs)
    fids, fw, fbufs = _route_dispatch(wl.logits, wl.x, wl.top_k)
    assert np.array_equal(fids, rids)
    assert np.array_equal(fw, w)
    _check_dispatch(rids, wl.x, wl.num_experts, fbufs)


@pytest.mark.parametrize("T,E,K,hidden", [
    (1, 8, 2, 64), (63, 8, 2, 4096), (65, 8, 2, 128), (1000, 64, 8, 256), (777, 256, 1, 8),
    (513, 16, 4, 100), (200, 3, 3, 24),
    # row copies over several 8-vector batches, the last one partial
    (130, 8, 2, 8200),
    # count matrices scanned in LDS (313 chunks x 8 experts) and by the scan
    # kernel (64 x 256; 1094 x 64, five chunks per scan thread)
    (20000, 8, 2, 64), (1025, 64, 8, 16), (4096, 256, 8, 16), (70000, 64, 2, 8)])
def test_route_dispatch_shapes(dev, T, E, K, hidden):
    rng = np.random.default_rng(T + E * 10 + K)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    x = rng.standard_normal((T, hidden)).astype(np.float16)
    ids, w = _route(logits, K)
    rids, rw = oracle.moe_route(logits, K)
    assert np.array_equal(ids, rids)
    assert np.abs(w - rw).max() <= 1e-6
    bufs = _dispatch(ids, x, E)
    _check_dispatch(ids, x, E, bufs)
    fids, fw, fbufs = _route_dispatch(logits, x, K)
    assert np.array_equal(fids, rids)
    assert np.array_equal(fw, w)
    _check_dispatch(rids, x, E, fbufs)


def test_route_ties_go_to_lower_index(dev):
    """Stable descending order (sampling/mod.rs:374): equal logits keep the
    lower expert index first."""
    rng = np.random.default_rng(3)
    T, E, K = 512, 8, 3
    logits = (np.round(rng.standard_normal((T, E)) * 2) / 2).astype(np.float32)  # many ties
    logits[0] = 1.0   # all equal: experts 0, 1, 2
    logits[1] = -np.inf
    logits[1, 5] = 0.0
    ids, w = _route(logits, K)
    rids, rw = oracle.moe_route(logits, K)
    assert list(ids[0]) == [0, 1, 2]
    assert ids[1, 0] == 5
    assert np.array_equal(ids, rids)
    assert np.abs(w[np.isfinite(rw)] - rw[np.isfinite(rw)]).max() <= 1e-6


def test_dispatch_index_only_and_dropped_ids(dev):
    rng = np.random.default_rng(4)
    T, E, K = 300, 8, 2
    ids = rng.integers(0, E, size=(T, K)).astype(np.int32)
    ids[::7, 1] = -1      # dropped entries
    ids[::11, 0] = E + 3  # out of range: dropped
    x = rng.standard_normal((T, 64)).astype(np.float16)
    bufs = _dispatch(ids, x, E, with_rows=False)
    _check_dispatch(ids, x, E, bufs, with_rows=False)
    bufs = _dispatch(ids, x, E, with_rows=True)
    _check_dispatch(ids, x, E, bufs, with_rows=True)


def test_dispatch_workspace_reuse(dev):
    """One workspace over calls of falling and rising sizes: nothing of an
    earlier call leaks into a later one."""
    rng = np.random.default_rng(6)
    E, K = 8, 2
    bufs = moe.DispatchBuffers.allocate(20000, E, K, 128)
    for T in (20000, 4096, 100, 17000, 20000, 2048):
        ids = rng.integers(0, E, size=(T, K)).astype(np.int32)
        x = rng.standard_normal((T, 128)).astype(np.float16)
        moe.moe_dispatch(DeviceArray.from_numpy(ids), DeviceArray.from_numpy(x), E, bufs)
        synchronize()
        counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, E)
        assert np.array_equal(bufs.offsets.numpy(), offsets)
        assert np.array_equal(bufs.inverse.numpy()[:T], inverse)
        n = int(offsets[-1])
        assert np.array_equal(bufs.x_perm.numpy()[:n].view(np.uint16), x[sorted_ids].view(np.uint16))


def test_dispatch_zero_tokens(dev):
    """No tokens: counts and offsets are written as zeros, nothing else."""
    E, K = 8, 2
    bufs = moe.DispatchBuffers.allocate(0, E, K, 64)
    bufs.counts.fill_byte(0x7F)
    bufs.offsets.fill_byte(0x7F)
    ids = DeviceArray((0, K), np.int32)
    moe.moe_dispatch(ids, DeviceArray((0, 64), np.float16), E, bufs)
    synchronize()
    assert bufs.counts.numpy().tolist() == [0] * E
    assert bufs.offsets.numpy().tolist() == [0] * (E + 1)
