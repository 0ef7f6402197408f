"""The lane reductions every kernel is built on, lane by lane against a
sequential float64 reference (the reference's butterflies are
paged_attention.cu:17-31, 32 lanes; here 64-lane waves), through
swiftllm_hip_wave_reduce_check, which runs the same inlined functions:

  max_over_kg / sum_over_kg  lanes l, l^16, l^32, l^48 (the softmax row max
                             and sum in the MFMA accumulator layout)
  wave_max / wave_sum        all 64 lanes (the split-K reduce)
  wave_inclusive_scan        64-lane prefix sum (dispatch offsets, item lists)

Bars: maxima and the integer scan are exact; a sum of n = 2^k terms by a
butterfly rounds k times, so |sum - exact| <= gamma_k * sum |x| with
gamma_k = k u / (1 - k u), u = 2^-24 (Higham, Accuracy and Stability of
Numerical Algorithms, 2nd ed., 4.2). Every lane of a group must return
bit-identical values: both lanes of a swap add the same pair.
"""

import numpy as np
import pytest

from swiftllm_amd import _lib
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, synchronize

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def _gamma(k):
    return k * U / (1 - k * U)


def _rows():
    rng = np.random.default_rng(17)
    rows = [rng.standard_normal((200, 64)).astype(np.float32)]
    for scale in (1e-30, 1e-3, 1e3, 1e30):
        rows.append((rng.standard_normal((20, 64)) * scale).astype(np.float32))
    special = np.zeros((12, 64), np.float32)
    special[0] = -np.inf                                   # a row no key reached
    special[1, ::2] = -np.inf                              # half the lanes masked
    special[1, 1::2] = rng.standard_normal(32)
    special[2] = 3.5                                       # ties everywhere
    special[3, :] = -0.0
    special[3, ::3] = 0.0                                  # signed zeros
    special[4] = np.where(np.arange(64) % 2 == 0, 1e8, -1e8)
    special[4, 5] = 1.0                                    # cancellation
    special[5] = np.float32(np.finfo(np.float32).tiny) * rng.integers(1, 5, 64)  # smallest normals
    special[6] = np.float32(1e-40) * rng.integers(1, 5, 64)                       # subnormals
    special[7] = np.arange(64, dtype=np.float32)           # max in the last lane
    special[8] = np.arange(64, dtype=np.float32)[::-1]     # max in lane 0
    special[9] = -np.inf
    special[9, 37] = -5.0                                  # one finite lane
    special[10] = rng.standard_normal(64).astype(np.float32)
    special[10, 16:] = -np.inf                             # only the first 16 lanes live
    special[11] = np.float32(3e38) / 64                    # a sum just below overflow
    rows.append(special)
    return np.concatenate(rows)


def _run(x, xi):
    n = x.shape[0]
    out = DeviceArray((n, 4, 64), np.float32)
    scan = DeviceArray((n, 64), np.int32)
    dx, dxi = DeviceArray.from_numpy(x), DeviceArray.from_numpy(xi)  # alive until the sync
    rc = _lib.lib().swiftllm_hip_wave_reduce_check(dx.ptr, dxi.ptr, n, out.ptr, scan.ptr, None)
    pa.check_status(rc)
    synchronize()
    return out.numpy(), scan.numpy()


def test_wave_reductions_lane_by_lane(dev):
    x = _rows()
    rng = np.random.default_rng(18)
    xi = rng.integers(-(1 << 20), 1 << 20, size=x.shape, dtype=np.int32)
    xi[0] = 1
    out, scan = _run(x, xi)
    x64 = x.astype(np.float64)
    groups = x64.reshape(-1, 4, 16)                        # [row][k][l % 16]: lane l % 16 + 16 k
    gmax = groups.max(axis=1)                              # [row][16]
    gsum = groups.sum(axis=1)
    gabs = np.abs(groups).sum(axis=1)
    for lane in range(64):
        got_max = out[:, 0, lane].astype(np.float64)
        got_sum = out[:, 1, lane].astype(np.float64)
        want_max = gmax[:, lane % 16]
        assert np.array_equal(got_max, want_max), f"max_over_kg lane {lane}"
        want_sum = gsum[:, lane % 16]
        fin = np.isfinite(want_sum)
        assert np.all(got_sum[~fin] == want_sum[~fin]), f"sum_over_kg lane {lane}: -inf groups"
        assert np.all(np.abs(got_sum[fin] - want_sum[fin]) <= _gamma(2) * gabs[fin, lane % 16]), \
            f"sum_over_kg lane {lane}"
    # every lane of a group holds the identical value
    for k in (16, 32, 48):
        assert np.array_equal(out[:, :2, :].view(np.uint32)[:, :, np.arange(64)],
                              out[:, :2, :].view(np.uint32)[:, :, np.arange(64) ^ k]), f"lanes l, l^{k}"
    wmax = x64.max(axis=1)
    wsum = x64.sum(axis=1)
    wabs = np.abs(x64).sum(axis=1)
    assert np.all(out[:, 2, :].view(np.uint32) == out[:, 2, :1].view(np.uint32))
    assert np.all(out[:, 3, :].view(np.uint32) == out[:, 3, :1].view(np.uint32))
    assert np.array_equal(out[:, 2, 0].astype(np.float64), wmax), "wave_max"
    fin = np.isfinite(wsum)
    assert np.all(out[~fin, 3, 0].astype(np.float64) == wsum[~fin]), "wave_sum: -inf rows"
    assert np.all(np.abs(out[fin, 3, 0].astype(np.float64) - wsum[fin]) <= _gamma(6) * wabs[fin]), "wave_sum"
    assert np.array_equal(scan, np.cumsum(xi, axis=1, dtype=np.int64).astype(np.int32)), "scan"


def test_exact_max_would_catch_a_wrong_partner(dev):
    """A butterfly with the wrong partner (l ^ 8 where l ^ 16 belongs) takes
    the maximum over lanes l, l ^ 8, l ^ 32, l ^ 40; on random rows that
    differs from the right group's in most lanes, so the exact check above
    tells them apart, and the library's output is the right one."""
    rng = np.random.default_rng(19)
    x = rng.standard_normal((64, 64)).astype(np.float32)
    out, _ = _run(x, np.zeros_like(x, dtype=np.int32))
    lanes = np.arange(64)
    right = np.max(np.stack([x[:, lanes ^ k] for k in (0, 16, 32, 48)]), axis=0)
    wrong = np.max(np.stack([x[:, lanes ^ k] for k in (0, 8, 32, 40)]), axis=0)
    assert (wrong != right).mean() > 0.3
    assert np.array_equal(out[:, 0, :], right)
