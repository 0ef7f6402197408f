"""swiftllm_hip_launch_paged_attention_v2_noalloc: split-K decode whose
scratch is the library's static device array instead of a caller workspace.

Through the C ABI, each call's output must equal, bit for bit, the output of
swiftllm_hip_launch_paged_attention_v2 with an allocated workspace on the
same inputs (the same kernels run; only the scratch address differs), and
stay within the attention tolerance of the fp64 oracle. Calls follow each
other on one stream, the later ones smaller, so each runs over the scratch
contents the previous one left. Sizes beyond the static scratch are refused.
The first test makes the process's first no-alloc call inside stream capture
(the device address of the static scratch is looked up on that call), so it
must stay first in this file, and this file must run after every other test
that could call the entry.
"""

import ctypes

import numpy as np
import pytest

import oracle
from helpers import assert_attention_close
from swiftllm_amd import _lib
from swiftllm_amd import paged_attention as pa
from swiftllm_amd import workloads
from swiftllm_amd._hip import DeviceArray, Graph, Stream

pytestmark = pytest.mark.gpu


class _Case:
    def __init__(self, w):
        self.w = w
        self.sh = w.shape
        self.q = DeviceArray.from_numpy(w.q)
        self.kc = DeviceArray.from_numpy(w.key_cache)
        self.vc = DeviceArray.from_numpy(w.value_cache)
        self.bt = DeviceArray.from_numpy(w.block_tables)
        self.ctx = DeviceArray.from_numpy(w.context_lens)

    def args(self):
        sh = self.sh
        return (self.q.ptr, self.kc.ptr, self.vc.ptr, self.bt.ptr, self.ctx.ptr,
                ctypes.c_float(self.w.scale), sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"],
                sh["head_dim"], sh["block_size"], sh["max_num_blocks_per_seq"])

    def noalloc(self, ps, stream):
        out = DeviceArray(self.w.q.shape, np.float16)
        out.fill_byte(0xFF)
        rc = _lib.lib().swiftllm_hip_launch_paged_attention_v2_noalloc(
            out.ptr, *self.args(), ps, self.sh["num_blocks"], stream.handle)
        assert rc == 0, _lib.last_error()
        return out

    def with_workspace(self, ps, stream):
        sh = self.sh
        out = DeviceArray(self.w.q.shape, np.float16)
        out.fill_byte(0xFF)
        nbytes = pa.paged_attention_v2_workspace_size(
            sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"], sh["head_dim"], sh["block_size"],
            sh["max_num_blocks_per_seq"], ps)
        ws = pa.workspace(nbytes, stream)
        rc = _lib.lib().swiftllm_hip_launch_paged_attention_v2(
            out.ptr, ws.ptr, nbytes, *self.args(), ps, sh["num_blocks"], stream.handle)
        assert rc == 0, _lib.last_error()
        return out, ws

    def ref(self):
        w = self.w
        return oracle.decode_f64(w.q, w.key_cache, w.value_cache, w.block_tables, w.context_lens,
                                 w.scale)


def test_noalloc_first_call_captured_in_a_graph(dev):
    """The first no-alloc call of the process is captured into a HIP graph.
    Three replays, each after an eager no-alloc call on other inputs that
    overwrites the shared scratch, must equal the workspace entry point's
    output bit for bit."""
    stream = Stream()
    case = _Case(workloads.decode_config(3, seed=33, ctx=4096, num_seqs=4))
    other = _Case(workloads.decode_config(1, seed=34, num_seqs=5))
    out = DeviceArray(case.w.q.shape, np.float16)
    status = []

    def enqueue():
        status.append(_lib.lib().swiftllm_hip_launch_paged_attention_v2_noalloc(
            out.ptr, *case.args(), 512, case.sh["num_blocks"], stream.handle))

    graph = Graph(stream, enqueue)
    assert status == [0], _lib.last_error()
    want, ws = case.with_workspace(512, stream)
    stream.synchronize()
    r = want.numpy()
    for rep in range(3):
        other.noalloc(64, stream)
        out.fill_byte(0xFF)
        graph.launch(stream)
        stream.synchronize()
        g = out.numpy()
        assert np.array_equal(g.view(np.uint16), r.view(np.uint16)), f"replay {rep} differs"
    assert_attention_close(g, case.ref(), "noalloc captured, config 3 heads, 4 x 4096 tokens")
    ws.free()


def test_noalloc_matches_workspace_entry_on_consecutive_calls(dev):
    """Config 3's heads at 16384 tokens in 512-token partitions (partition
    streams: 8.4 MB of partial outputs and 8.7 MB of boundary slots in the
    scratch, the workgroup reduce over 32 partitions), then a smaller batch
    (config 1's shape) at 64-token partitions, then the small batch again in
    balanced mode: each bit-equal to the workspace entry point and within the
    oracle's tolerance."""
    stream = Stream()
    big = _Case(workloads.decode_config(3, seed=31, ctx=16384))
    small = _Case(workloads.decode_config(1, seed=32, num_seqs=7))
    calls = [(big, 512), (small, 64), (small, 0)]
    for case, ps in calls:
        got = case.noalloc(ps, stream)
        want, ws = case.with_workspace(ps, stream)
        stream.synchronize()
        g, r = got.numpy(), want.numpy()
        assert np.array_equal(g.view(np.uint16), r.view(np.uint16)), \
            f"noalloc differs from the workspace entry (S={case.sh['num_seqs']}, ps={ps})"
        assert_attention_close(g, case.ref(), f"noalloc S={case.sh['num_seqs']} ps={ps}")
        ws.free()


def test_noalloc_refuses_sizes_beyond_its_scratch(dev):
    """256 sequences x 64 heads x 4096 partitions of 16 tokens need far more
    than 64 MiB; the call returns InvalidParameter before any launch."""
    q = DeviceArray((256, 64, 128), np.float16)
    out = DeviceArray((256, 64, 128), np.float16)
    bt = DeviceArray((256, 4096), np.int32)
    ctx = DeviceArray((256,), np.int32)
    need = pa.paged_attention_v2_workspace_size(256, 64, 8, 128, 16, 4096, 16)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    rc = _lib.lib().swiftllm_hip_launch_paged_attention_v2_noalloc(
        out.ptr, q.ptr, q.ptr, q.ptr, bt.ptr, ctx.ptr, ctypes.c_float(0.1), 256, 64, 8, 128, 16,
        4096, 16, 0, None)
    assert rc == pa.InvalidParameter.code
    assert "static scratch" in _lib.last_error()[1]
