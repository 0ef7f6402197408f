"""copy_blocks and swap_blocks on the GPU, bit-exact against the oracle
(oracle.copy_blocks / oracle.swap_blocks) on tagged pools: the drop-in
launcher of paged_attention.cu:302-327, its bounded status twin, the layered
form of bindings.rs:200-223, and swaps between device memory and pinned host
memory (bindings.rs:225-242)."""

import numpy as np
import pytest

import oracle
from swiftllm_amd import _lib
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, HostArray, synchronize

pytestmark = pytest.mark.gpu


def _pool(rng, NB, Hkv, D, BS):
    return rng.integers(1, 65000, size=(NB, Hkv, D, BS), dtype=np.uint16)


def _mapping(rng, NB, n, holes=0):
    """n disjoint pairs: sources and destinations drawn without repetition."""
    ids = rng.permutation(NB)[:2 * n]
    m = np.stack([ids[:n], ids[n:]], axis=1).astype(np.int64)
    if holes:
        m[rng.choice(n, size=holes, replace=False), rng.integers(0, 2)] = -1
    return m


@pytest.mark.parametrize("Hkv,D,BS,NB,pairs", [
    (8, 128, 16, 64, 20),    # Llama-3-8B layer: 32 KiB blocks, two chunks per block
    (2, 64, 16, 9, 4),
    (1, 5, 3, 10, 3),        # 30-byte blocks: the byte path
])
def test_launch_copy_blocks_dropin(dev, Hkv, D, BS, NB, pairs):
    rng = np.random.default_rng(Hkv * 100 + D)
    kc, vc = _pool(rng, NB, Hkv, D, BS), _pool(rng, NB, Hkv, D, BS)
    m = _mapping(rng, NB, pairs, holes=1)
    kd, vd, md = DeviceArray.from_numpy(kc), DeviceArray.from_numpy(vc), DeviceArray.from_numpy(m)
    _lib.lib().launch_copy_blocks(md.ptr, kd.ptr, vd.ptr, pairs, Hkv, D, BS, None)
    assert _lib.lib().swiftllm_hip_last_error() == 0
    synchronize()
    oracle.copy_blocks([kc], [vc], m)
    assert np.array_equal(kd.numpy(), kc)
    assert np.array_equal(vd.numpy(), vc)


def test_copy_blocks_bounded_skips_out_of_pool(dev):
    rng = np.random.default_rng(3)
    NB, Hkv, D, BS = 16, 8, 128, 16
    kc, vc = _pool(rng, NB, Hkv, D, BS), _pool(rng, NB, Hkv, D, BS)
    m = np.array([[1, 2], [3, NB + 5], [NB, 4], [6, 7]], np.int64)
    kd, vd, md = DeviceArray.from_numpy(kc), DeviceArray.from_numpy(vc), DeviceArray.from_numpy(m)
    pa.launch_copy_blocks(md, kd, vd, len(m), Hkv, D, BS, num_blocks=NB)
    synchronize()
    oracle.copy_blocks([kc], [vc], m[[0, 3]])
    assert np.array_equal(kd.numpy(), kc)
    assert np.array_equal(vd.numpy(), vc)


@pytest.mark.parametrize("layers", [1, 3, 70])
def test_copy_blocks_layered(dev, layers):
    """bindings.rs:200-223: one mapping over the K and V caches of every
    layer (70 layers take three launches of up to 32 layers)."""
    rng = np.random.default_rng(layers)
    NB, Hkv, D, BS = 12, 2, 64, 16
    kcs = [_pool(rng, NB, Hkv, D, BS) for _ in range(layers)]
    vcs = [_pool(rng, NB, Hkv, D, BS) for _ in range(layers)]
    m = _mapping(rng, NB, 5)
    kds = [DeviceArray.from_numpy(k) for k in kcs]
    vds = [DeviceArray.from_numpy(v) for v in vcs]
    pa.copy_blocks(kds, vds, DeviceArray.from_numpy(m), len(m), Hkv, D, BS)
    synchronize()
    oracle.copy_blocks(kcs, vcs, m)
    for l in range(layers):
        assert np.array_equal(kds[l].numpy(), kcs[l]), l
        assert np.array_equal(vds[l].numpy(), vcs[l]), l


def test_copy_blocks_no_pairs(dev):
    rng = np.random.default_rng(9)
    kc = _pool(rng, 4, 2, 64, 16)
    kd = DeviceArray.from_numpy(kc)
    pa.copy_blocks([kd], [kd], DeviceArray((2,), np.int64), 0, 2, 64, 16)
    synchronize()
    assert np.array_equal(kd.numpy(), kc)


@pytest.mark.parametrize("direction", ["d2h", "h2d", "d2d", "h2h"])
@pytest.mark.parametrize("block_bytes", [32768, 4096 + 16, 1000 + 6])
def test_swap_blocks(dev, direction, block_bytes):
    rng = np.random.default_rng(block_bytes)
    NS, ND, pairs = 24, 20, 9
    src_np = rng.integers(0, 256, size=NS * block_bytes, dtype=np.uint8)
    dst_np = rng.integers(0, 256, size=ND * block_bytes, dtype=np.uint8)
    m = np.stack([rng.permutation(NS)[:pairs], rng.permutation(ND)[:pairs]], axis=1).astype(np.int64)
    m[4, 0] = -1

    def make(arr, host):
        if host:
            h = HostArray(arr.shape, arr.dtype)
            h.array()[...] = arr
            return h
        return DeviceArray.from_numpy(arr)

    src = make(src_np, direction[0] == "h")
    dst = make(dst_np, direction[2] == "h")
    md = HostArray(m.shape, np.int64) if direction == "h2h" else DeviceArray.from_numpy(m)
    if isinstance(md, HostArray):
        md.array()[...] = m
    pa.swap_blocks(src, dst, md, pairs, block_bytes)
    synchronize()
    got = dst.array().copy() if isinstance(dst, HostArray) else dst.numpy()
    oracle.swap_blocks(src_np, dst_np, m, block_bytes)
    assert np.array_equal(got, dst_np)


def test_swap_blocks_bounded(dev):
    rng = np.random.default_rng(5)
    nb, NS, ND = 512, 6, 4
    src_np = rng.integers(0, 256, size=NS * nb, dtype=np.uint8)
    dst_np = rng.integers(0, 256, size=ND * nb, dtype=np.uint8)
    m = np.array([[0, 1], [NS, 2], [2, ND], [5, 3]], np.int64)
    src, dst = DeviceArray.from_numpy(src_np), DeviceArray.from_numpy(dst_np)
    pa.launch_swap_blocks(src, dst, DeviceArray.from_numpy(m), len(m), nb, src_blocks=NS,
                          dst_blocks=ND)
    synchronize()
    oracle.swap_blocks(src_np, dst_np, m[[0, 3]], nb)
    assert np.array_equal(dst.numpy(), dst_np)
