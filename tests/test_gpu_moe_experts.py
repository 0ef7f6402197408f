"""MoE expert computation on the GPU against the float64 oracle: the grouped
expert GEMM (plain and with the fused SwiGLU gate), the weighted combine,
and the whole MoeMlp chain (route, dispatch, gated GEMM, down GEMM,
combine) at a small Mixtral-like shape.

Tolerance: fp16 outputs of fp32 accumulation against float64 on the same
fp16 inputs: |gpu - ref| <= 2^-10 |ref| + 1e-3 rms(ref) (one fp16 rounding
plus fp32 accumulation; an indexing mistake is off by O(rms)). The combine is
held to one fp16 ulp plus the error bound of its fp32 chain, and > 99% of its
outputs to the correctly rounded value."""

import numpy as np
import pytest

import oracle
from helpers import assert_gemm_close as _close
from helpers import expert_offsets as _offsets
from swiftllm_amd import moe, workloads
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gated", [False, True])
@pytest.mark.parametrize("E,m_total,n,k", [
    (4, 300, 256, 128),
    (8, 1000, 512, 192),
    (1, 257, 256, 64),       # one expert, a 1-row tail tile
    (3, 0, 256, 64),
    (5, 40, 256, 128),       # 40 rows: no main-grid tile at all, the thin kernel only
])
def test_expert_gemm(dev, gated, E, m_total, n, k):
    """Tiles of 256 rows; columns in tiles of 256 (plain) or 128 (gated)."""
    rng = np.random.default_rng(E * 1000 + m_total + gated)
    offs = _offsets(rng, E, m_total, empty=(1,) if E > 2 else ())
    a = (rng.standard_normal((max(m_total, 1), k)) * 0.5).astype(np.float16)[:m_total]
    w = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16)
    w2 = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16) if gated else None
    ad = DeviceArray.from_numpy(a) if m_total else DeviceArray((0, k), np.float16)
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(ad, DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None,
                        DeviceArray.from_numpy(offs), c)
    synchronize()
    if m_total:
        _close(c.numpy().astype(np.float64), oracle.moe_expert_gemm(a, w, w2, offs),
               f"gemm gated={gated} E{E} M{m_total}")


@pytest.mark.parametrize("gated,n,k", [(False, 256, 320), (True, 384, 320), (False, 512, 64),
                                       (True, 128, 128)])
def test_expert_gemm_thin_tails(dev, gated, n, k):
    """Expert row counts around the thin-tail limit: tails of at most 128 rows
    go to the thin kernel (up to four 32-row tiles), longer ones to a 256-row
    tile; an expert of 257 rows is one whole tile plus a 1-row tail, 384 a
    whole tile plus a 128-row tail, 385 two tiles. Every output row is
    checked against the oracle."""
    counts = [0, 1, 31, 32, 33, 64, 65, 100, 128, 129, 256, 257, 320, 384, 385, 528, 16]
    rng = np.random.default_rng(n + k + gated)
    E = len(counts)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    m_total = int(offs[-1])
    a = (rng.standard_normal((m_total, k)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16)
    w2 = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16) if gated else None
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(DeviceArray.from_numpy(a), DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None, DeviceArray.from_numpy(offs), c)
    synchronize()
    _close(c.numpy().astype(np.float64), oracle.moe_expert_gemm(a, w, w2, offs),
           f"thin tails gated={gated} n={n} k={k}")


@pytest.mark.parametrize("gated", [False, True])
def test_expert_gemm_many_experts(dev, gated):
    """160 experts: the main kernel's per-expert tile table is a wave scan in
    chunks of 64 experts with a carry, so three chunks (the last partial)
    meet here; counts from 0 to 600 rows give most experts a thin tail and
    some whole tiles, at expert indices past 64 and 128."""
    rng = np.random.default_rng(160 + gated)
    E, n, k = 160, (128 if gated else 256), 128
    counts = rng.integers(0, 40, E)
    counts[rng.choice(E, 12, replace=False)] = rng.integers(200, 600, 12)
    counts[[70, 150]] = [300, 513]   # whole tiles past the first and second chunk
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    m_total = int(offs[-1])
    a = (rng.standard_normal((m_total, k)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16)
    w2 = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16) if gated else None
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(DeviceArray.from_numpy(a), DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None, DeviceArray.from_numpy(offs), c)
    synchronize()
    _close(c.numpy().astype(np.float64), oracle.moe_expert_gemm(a, w, w2, offs),
           f"160 experts gated={gated} rows={m_total}")


@pytest.mark.parametrize("gated", [False, True])
def test_expert_gemm_decode_batch(dev, gated):
    """A decode step's MoE: 64 tokens, top-2 of 8 experts, so every expert
    holds a few rows and the whole GEMM runs in the thin kernel (k 4096,
    n 1024)."""
    rng = np.random.default_rng(64 + gated)
    E, n, k = 8, 1024, 4096
    ids = np.stack([rng.choice(E, 2, replace=False) for _ in range(64)])
    counts = np.bincount(ids.ravel(), minlength=E)
    offs = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    m_total = int(offs[-1])
    a = (rng.standard_normal((m_total, k)) * 0.5).astype(np.float16)
    w = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16)
    w2 = (rng.standard_normal((E, n, k)) / np.sqrt(k)).astype(np.float16) if gated else None
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(DeviceArray.from_numpy(a), DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None, DeviceArray.from_numpy(offs), c)
    synchronize()
    _close(c.numpy().astype(np.float64), oracle.moe_expert_gemm(a, w, w2, offs),
           f"decode batch gated={gated} counts {list(counts)}")


@pytest.mark.parametrize("T,K,hidden", [(500, 2, 4096), (300, 1, 4104), (257, 3, 520), (64, 4, 1032),
                                        (33, 5, 4096), (100, 6, 8), (129, 8, 2056), (40, 9, 264)])
def test_combine(dev, T, K, hidden):
    """Top-k 1-4, 6 and 8 take the compile-time kernels, 5 and 9 the generic
    one; hidden sizes that leave partial unroll groups. Entries of -1 and
    past the last row of y give no term; row 0 of y holds NaN and no valid
    entry points to it, which the masked loads of those entries read.

    Bound: the fp32 chain of K fused multiply-adds is within K 2^-24
    sum_k |w_k y_k| of the exact sum, and its fp16 rounding within one fp16
    ulp of the result. Where the terms cancel to a subnormal fp16 value the
    fp32 chain alone can be several fp16 ulps off (the CPU emulation of the
    chain is 2 ulps off at one element of the top-8 case), while an indexing
    mistake is off by O(1)."""
    rng = np.random.default_rng(21 + K)
    y = rng.standard_normal((T * K, hidden)).astype(np.float16)
    wts = rng.random((T, K)).astype(np.float32)
    inv = rng.permutation(T * K).reshape(T, K).astype(np.int32)
    inv[::13, K - 1] = -1
    inv[5::17, 0] = T * K + 3
    inv[inv == 0] = -1
    y[0] = np.nan
    out = DeviceArray((T, hidden), np.float16)
    out.fill_byte(0xFF)
    moe.moe_combine(DeviceArray.from_numpy(y), DeviceArray.from_numpy(wts),
                    DeviceArray.from_numpy(inv), out)
    synchronize()
    got = out.numpy()
    inv_ref = np.where(inv < T * K, inv, -1)
    exact = oracle.moe_combine(y, wts, inv_ref)
    ref = exact.astype(np.float16)
    assert not np.isnan(got).any()
    mag = oracle.moe_combine(np.abs(np.nan_to_num(y)), wts, inv_ref)
    ulp = np.spacing(np.maximum(np.abs(got), np.abs(ref))).astype(np.float64)
    err = np.abs(got.astype(np.float64) - exact)
    assert (err <= ulp + K * 2.0 ** -24 * mag).all(), f"max err {err.max():.3g}"
    assert np.mean(got.view(np.uint16) == ref.view(np.uint16)) > 0.99


@pytest.mark.parametrize("T", [96, 1100])
def test_moe_mlp_chain(dev, T):
    """MoeMlp from router logits: top-2 of 8 experts, hidden 256,
    intermediate 512. 96 tokens leave every expert a tail of at most 64 rows
    (the thin kernel only); 1100 give whole tiles and longer tails as well.

    Each stage is held to the oracle on the GPU's own input to that stage:
    routing and dispatch bit-exact, the gated GEMM on the permuted rows, the
    down GEMM on the GPU's fp16 intermediate, the combine on the GPU's expert
    outputs. Against an oracle chain that rounds its own float64
    intermediate instead, about 0.1% of the intermediate's elements round to
    the neighbouring fp16 value, and the down GEMM carries those one-ulp
    differences into its outputs: that compares two roundings, not the
    kernels. An indexing mistake in any stage is off by O(rms) in that
    stage's check."""
    rng = np.random.default_rng(22)
    hidden, I, E, K = 256, 512, 8, 2
    x = rng.standard_normal((T, hidden)).astype(np.float16)
    logits = rng.standard_normal((T, E)).astype(np.float32)
    wg = (rng.standard_normal((E, I, hidden)) / np.sqrt(hidden)).astype(np.float16)
    wu = (rng.standard_normal((E, I, hidden)) / np.sqrt(hidden)).astype(np.float16)
    wd = (rng.standard_normal((E, hidden, I)) / np.sqrt(I)).astype(np.float16)
    mlp = moe.MoeMlp(E, K, DeviceArray.from_numpy(wg), DeviceArray.from_numpy(wu),
                     DeviceArray.from_numpy(wd))
    out = mlp.forward(DeviceArray.from_numpy(logits), DeviceArray.from_numpy(x))
    synchronize()
    b = mlp.buffers(T, hidden)
    d = b["dispatch"]
    ids, w = oracle.moe_route(logits, K)
    counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(ids, E)
    assert np.array_equal(b["ids"].numpy(), ids)
    assert np.abs(b["weights"].numpy() - w).max() <= 1e-6
    assert np.array_equal(d.offsets.numpy(), offsets)
    assert np.array_equal(d.inverse.numpy(), inverse)
    h = b["h"].numpy()
    _close(h.astype(np.float64), oracle.moe_expert_gemm(x[sorted_ids], wg, wu, offsets),
           f"T={T} gated GEMM")
    y = b["y"].numpy()
    _close(y.astype(np.float64), oracle.moe_expert_gemm(h, wd, None, offsets), f"T={T} down GEMM")
    _close(out.numpy().astype(np.float64), oracle.moe_combine(y, b["weights"].numpy(), inverse),
           f"T={T} combine")


def _sample_rows(rng, offs, tile=256, per_tile=2):
    """Rows to check against the float64 oracle: for every expert with rows,
    its first and last row and `per_tile` random rows of each 256-row tile,
    so every (row tile, column tile) pair of the grid is covered."""
    rows = []
    for e in range(len(offs) - 1):
        r0, r1 = int(offs[e]), int(offs[e + 1])
        if r1 <= r0:
            continue
        rows += [r0, r1 - 1]
        for t0 in range(r0, r1, tile):
            t1 = min(t0 + tile, r1)
            rows += [int(x) for x in rng.integers(t0, t1, per_tile)]
    return np.unique(np.array(rows, np.int64))


@pytest.mark.parametrize("gated,n,k", [(True, 14336, 4096), (False, 4096, 14336)])
def test_expert_gemm_mixtral_size(dev, gated, n, k):
    """The sizes bench config 8 runs (Mixtral-8x7B layer, 4096 tokens top-2):
    gated k 4096 -> n 14336 and down k 14336 -> n 4096 over m_total 8192
    rows in 8 uneven experts, expert 5 empty, a different weight for every
    expert. That is 56 / 16 column tiles, the 64- and 224-step k loops and
    the XCD super-tile remap over hundreds of tiles, none of which the small
    shapes reach.

    Checks: every output is written (the output starts as NaN); sampled rows
    from every row tile, all n columns, against the float64 oracle; and for
    the plain GEMM every row through a random-sign projection:
    c_row . v = a_row . (W_e^T v) exactly, and the rounding of the n fp16
    outputs (each within 2^-11 of its value) moves c_row . v by a Rademacher
    sum of standard deviation <= 2^-11 ||c_row||, held to 7 of those (plus
    the fp32 accumulation) where one wrong element moves it by O(rms)."""
    E, m_total = 8, 8192
    rng = np.random.default_rng(8 + gated)
    offs = _offsets(rng, E, m_total, empty=(5,))
    a = workloads._normal_f16(rng, (m_total, k), 0.5)
    w = workloads.expert_weights(rng, E, n, k)
    w2 = workloads.expert_weights(rng, E, n, k) if gated else None
    c = DeviceArray((m_total, n), np.float16)
    c.fill_byte(0xFF)
    moe.moe_expert_gemm(DeviceArray.from_numpy(a), DeviceArray.from_numpy(w),
                        DeviceArray.from_numpy(w2) if gated else None,
                        DeviceArray.from_numpy(offs), c)
    synchronize()
    got = c.numpy()
    assert np.isfinite(got).all(), "an output was not written (still NaN)"

    rows = _sample_rows(rng, offs)
    sub_counts = [int(((rows >= offs[e]) & (rows < offs[e + 1])).sum()) for e in range(E)]
    sub_offs = np.concatenate([[0], np.cumsum(sub_counts)]).astype(np.int32)
    ref = oracle.moe_expert_gemm(a[rows], w, w2, sub_offs)
    _close(got[rows].astype(np.float64), ref, f"gemm gated={gated} n{n} k{k} sampled rows")

    if not gated:
        v = rng.choice([-1.0, 1.0], size=n)
        g = got.astype(np.float64)
        lhs = g @ v
        rms = float(np.sqrt(np.mean(ref ** 2)))
        for e in range(E):
            r0, r1 = int(offs[e]), int(offs[e + 1])
            if r1 <= r0:
                continue
            rhs = a[r0:r1].astype(np.float64) @ (w[e].astype(np.float64).T @ v)
            sigma = 2.0 ** -11 * np.linalg.norm(g[r0:r1], axis=1) + 1e-4 * rms * np.sqrt(n)
            worst = float((np.abs(lhs[r0:r1] - rhs) - 7 * sigma).max())
            assert worst <= 0, f"expert {e}: projection off by {worst:.3e} beyond 7 sigma"
