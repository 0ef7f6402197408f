"""Shared helpers for the tests: running the library on numpy inputs, the
attention tolerance of the decode path and the expert GEMM's tolerance."""

from __future__ import annotations

import numpy as np

from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, synchronize

# Attention tolerance against the fp64 oracle (fp16 in/out, fp32 accumulate):
# max |out - ref| <= 2e-3 and max |out - ref| / max(|ref|, 1e-3) <= 1e-2.
ATOL = 2e-3
RTOL = 1e-2
REL_FLOOR = 1e-3


def attention_errors(out, ref):
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    diff = np.abs(out - ref)
    max_abs = float(diff.max()) if diff.size else 0.0
    max_rel = float((diff / np.maximum(np.abs(ref), REL_FLOOR)).max()) if diff.size else 0.0
    norm_rel = float(np.linalg.norm(out - ref) / max(np.linalg.norm(ref), 1e-30)) if diff.size else 0.0
    return max_abs, max_rel, norm_rel


def assert_attention_close(out, ref, what=""):
    assert np.all(np.isfinite(np.asarray(out, dtype=np.float64))), f"{what}: non-finite output"
    max_abs, max_rel, norm_rel = attention_errors(out, ref)
    assert max_abs <= ATOL and max_rel <= RTOL, (
        f"{what}: max_abs={max_abs:.3e} (<= {ATOL}) max_rel={max_rel:.3e} (<= {RTOL}) "
        f"norm_rel={norm_rel:.3e}")
    return max_abs, max_rel, norm_rel


def assert_gemm_close(gpu, ref, what=""):
    """Expert GEMM tolerance: fp16 outputs of fp32 accumulation against
    float64 on the same fp16 inputs, |gpu - ref| <= 2^-10 |ref| + 1e-3
    rms(ref) (one fp16 rounding plus fp32 accumulation; an indexing mistake
    is off by O(rms))."""
    gpu = np.asarray(gpu, np.float64)
    assert np.all(np.isfinite(gpu)), what
    rms = float(np.sqrt(np.mean(ref ** 2))) if ref.size else 0.0
    err = np.abs(gpu - ref)
    bound = 2.0 ** -10 * np.abs(ref) + 1e-3 * rms
    worst = float((err - bound).max()) if err.size else -1.0
    assert worst <= 0, f"{what}: max err {err.max():.3e}, rms {rms:.3e}"


def expert_offsets(rng, E, m_total, empty=()):
    """Offsets of E experts over m_total rows cut at random points; the rows
    of each expert in `empty` move to the next one."""
    cuts = np.sort(rng.integers(0, m_total + 1, size=E - 1))
    counts = np.diff(np.concatenate([[0], cuts, [m_total]]))
    for e in empty:
        counts[(e + 1) % E] += counts[e]
        counts[e] = 0
    return np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)


class DeviceWorkload:
    """A decode workload uploaded to the device."""

    def __init__(self, w):
        self.w = w
        self.q = DeviceArray.from_numpy(w.q)
        self.kc = DeviceArray.from_numpy(w.key_cache)
        self.vc = DeviceArray.from_numpy(w.value_cache)
        self.bt = DeviceArray.from_numpy(w.block_tables)
        self.ctx = DeviceArray.from_numpy(w.context_lens)
        self.out = DeviceArray(w.q.shape, np.float16)

    def run(self, variant="v2", partition_size=None, bounded=True):
        w, sh = self.w, self.w.shape
        nb = sh["num_blocks"] if bounded else 0
        self.out.fill_byte(0xFF)  # NaN pattern: every output element must be written
        if variant == "v1":
            pa.paged_attention_v1(self.out, self.q, self.kc, self.vc, self.bt, self.ctx, w.scale,
                                  sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"],
                                  sh["block_size"], sh["max_num_blocks_per_seq"], num_blocks=nb)
        elif variant == "v2":
            ps = w.partition_size if partition_size is None else partition_size
            need = pa.paged_attention_v2_workspace_size(
                sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
                sh["max_num_blocks_per_seq"], ps)
            if getattr(self, "_ws", None) is None or self._ws.nbytes < need:
                self._ws = pa.workspace(need)
            pa.paged_attention_v2(self.out, self._ws, self.q, self.kc, self.vc, self.bt, self.ctx,
                                  w.scale, sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"],
                                  sh["head_dim"], sh["block_size"], sh["max_num_blocks_per_seq"], ps,
                                  num_blocks=nb)
        elif variant == "decode":
            params = pa.PagedAttentionParams(
                sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
                w.scale, sh["max_num_blocks_per_seq"] * sh["block_size"])
            pa.paged_attention_decode(self.out, self.q, self.kc, self.vc, self.bt, self.ctx, params)
        else:
            raise ValueError(variant)
        synchronize()
        return self.out.numpy()
