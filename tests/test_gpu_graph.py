"""The hot path inside a HIP graph: a ragged decode step (cache write, then
single-pass, balanced and 512-token split-K decode, the last as partition
streams at this batch size), the fused MoE route + dispatch, and the
whole MoE layer (MoeMlp.forward: dispatch, expert GEMMs with their thin
tails, combine) are captured once and replayed several times, with new inputs uploaded and the
program's own eager work and synchronisation between replays; every replay
must equal the eager run on the same inputs bit for bit (the kernels are
deterministic), and the decode outputs also meet the attention tolerance."""

import numpy as np
import pytest

import oracle
from helpers import assert_attention_close
from swiftllm_amd import moe, workloads
from swiftllm_amd import paged_attention as pa
from swiftllm_amd._hip import DeviceArray, Graph, Stream, synchronize

pytestmark = pytest.mark.gpu


class _Step:
    """Device buffers of one decode step and the calls that run it."""

    def __init__(self, w):
        sh = w.shape
        self.sh = sh
        self.w = w
        self.q = DeviceArray.from_numpy(w.q)
        self.kc = DeviceArray.from_numpy(w.key_cache)
        self.vc = DeviceArray.from_numpy(w.value_cache)
        self.bt = DeviceArray.from_numpy(w.block_tables)
        self.ctx = DeviceArray.from_numpy(w.context_lens)
        self.nk = DeviceArray.from_numpy(w.new_key)
        self.nv = DeviceArray.from_numpy(w.new_value)
        self.slots = DeviceArray.from_numpy(w.slot_mapping)
        self.o1 = DeviceArray(w.q.shape, np.float16)
        self.o2 = DeviceArray(w.q.shape, np.float16)
        self.o3 = DeviceArray(w.q.shape, np.float16)
        need = pa.paged_attention_v2_workspace_size(sh["num_seqs"], sh["num_heads"],
                                                    sh["num_kv_heads"], sh["head_dim"], 16,
                                                    sh["max_num_blocks_per_seq"], 0)
        self.ws = DeviceArray((need // 4 + 1,), np.uint32)
        need = pa.paged_attention_v2_workspace_size(sh["num_seqs"], sh["num_heads"],
                                                    sh["num_kv_heads"], sh["head_dim"], 16,
                                                    sh["max_num_blocks_per_seq"], 512)
        self.ws3 = DeviceArray((need // 4 + 1,), np.uint32)

    def enqueue(self, stream):
        w, sh = self.w, self.sh
        S, H, Hkv, D, MB, NB = (sh["num_seqs"], sh["num_heads"], sh["num_kv_heads"],
                                sh["head_dim"], sh["max_num_blocks_per_seq"], sh["num_blocks"])
        pa.launch_reshape_and_cache(self.nk, self.nv, self.kc, self.vc, self.slots, S, Hkv, D, 16,
                                    num_blocks=NB, stream=stream)
        pa.paged_attention_v1(self.o1, self.q, self.kc, self.vc, self.bt, self.ctx, w.scale, S, H,
                              Hkv, D, 16, MB, num_blocks=NB, stream=stream)
        pa.paged_attention_v2(self.o2, self.ws, self.q, self.kc, self.vc, self.bt, self.ctx,
                              w.scale, S, H, Hkv, D, 16, MB, 0, num_blocks=NB, stream=stream)
        pa.paged_attention_v2(self.o3, self.ws3, self.q, self.kc, self.vc, self.bt, self.ctx,
                              w.scale, S, H, Hkv, D, 16, MB, 512, num_blocks=NB, stream=stream)

    def upload(self, rng):
        """New query and new-token K/V (same shapes and slots)."""
        w = self.w
        for dev, host in ((self.q, w.q), (self.nk, w.new_key), (self.nv, w.new_value)):
            arr = rng.standard_normal(host.shape).astype(np.float16)
            host[...] = arr
            dev.upload(arr)


def test_decode_step_graph_replays_match_eager(dev):
    w = workloads.decode_config(4, seed=31, num_seqs=64)
    step = _Step(w)
    stream = Stream()
    graph = Graph(stream, lambda: step.enqueue(stream))
    rng = np.random.default_rng(32)
    eager = _Step(w)   # same cache contents; its own buffers
    for rep in range(3):
        step.upload(rng)
        for dev, host in ((eager.q, w.q), (eager.nk, w.new_key), (eager.nv, w.new_value)):
            dev.upload(host)
        synchronize()
        graph.launch(stream)
        stream.synchronize()
        eager.enqueue(stream)        # eager work between replays
        stream.synchronize()
        for a, b in ((step.o1, eager.o1), (step.o2, eager.o2), (step.o3, eager.o3)):
            assert np.array_equal(a.numpy().view(np.uint16), b.numpy().view(np.uint16)), rep
        # and the result is right: the oracle on the cache the step wrote
        kc, vc = step.kc.numpy(), step.vc.numpy()
        ref = oracle.decode_f64(w.q, kc, vc, w.block_tables, w.context_lens, w.scale)
        assert_attention_close(step.o1.numpy(), ref, f"graph replay {rep} v1")
        assert_attention_close(step.o2.numpy(), ref, f"graph replay {rep} balanced")
        assert_attention_close(step.o3.numpy(), ref, f"graph replay {rep} split-K 512")


def test_moe_route_dispatch_graph_replays_match_eager(dev):
    wl = workloads.moe_config(seed=33, num_tokens=1024, hidden=256)
    T, hidden = wl.x.shape
    E, K = wl.num_experts, wl.top_k
    logits, x = DeviceArray.from_numpy(wl.logits), DeviceArray.from_numpy(wl.x)
    ids, wts = DeviceArray((T, K), np.int32), DeviceArray((T, K), np.float32)
    bufs = moe.DispatchBuffers.allocate(T, E, K, hidden)
    stream = Stream()
    graph = Graph(stream, lambda: moe.moe_route_dispatch(logits, x, K, ids, wts, bufs, stream))
    rng = np.random.default_rng(34)
    for rep in range(3):
        lg = rng.standard_normal((T, E)).astype(np.float32)
        xx = rng.standard_normal((T, hidden)).astype(np.float16)
        logits.upload(lg)
        x.upload(xx)
        synchronize()
        graph.launch(stream)
        stream.synchronize()
        rids, rw = oracle.moe_route(lg, K)
        counts, offsets, inverse, sorted_ids = oracle.moe_dispatch(rids, E)
        assert np.array_equal(ids.numpy(), rids), rep
        assert np.abs(wts.numpy() - rw).max() <= 1e-6
        assert np.array_equal(bufs.offsets.numpy(), offsets)
        assert np.array_equal(bufs.inverse.numpy(), inverse)
        assert np.array_equal(bufs.x_perm.numpy().view(np.uint16), xx[sorted_ids].view(np.uint16))


def test_moe_mlp_graph_replays_match_eager(dev):
    """MoeMlp.forward whole: route + dispatch, the gated and the down expert
    GEMM (main grid and thin tails: 1100 tokens give every expert a whole
    256-row tile and a short tail) and the combine, captured once; each of
    three replays on new router logits and activations equals the eager
    forward on the same inputs bit for bit."""
    rng = np.random.default_rng(35)
    T, hidden, I, E, K = 1100, 256, 512, 8, 2
    wg = (rng.standard_normal((E, I, hidden)) / np.sqrt(hidden)).astype(np.float16)
    wu = (rng.standard_normal((E, I, hidden)) / np.sqrt(hidden)).astype(np.float16)
    wd = (rng.standard_normal((E, hidden, I)) / np.sqrt(I)).astype(np.float16)
    mlp = moe.MoeMlp(E, K, DeviceArray.from_numpy(wg), DeviceArray.from_numpy(wu),
                     DeviceArray.from_numpy(wd))
    logits = DeviceArray((T, E), np.float32)
    x = DeviceArray((T, hidden), np.float16)
    logits.upload(rng.standard_normal((T, E)).astype(np.float32))
    x.upload(rng.standard_normal((T, hidden)).astype(np.float16))
    stream = Stream()
    mlp.forward(logits, x, stream)   # buffers exist before the capture
    stream.synchronize()
    out = {}
    graph = Graph(stream, lambda: out.setdefault("dev", mlp.forward(logits, x, stream)))
    tails = []
    for rep in range(3):
        logits.upload(rng.standard_normal((T, E)).astype(np.float32))
        x.upload(rng.standard_normal((T, hidden)).astype(np.float16))
        synchronize()
        eager = mlp.forward(logits, x, stream)
        stream.synchronize()
        ref = eager.numpy()
        counts = mlp.buffers(T, hidden)["dispatch"].counts.numpy()
        tails.append(int(((counts % 256 > 0) & (counts % 256 <= 64)).sum()))
        out["dev"].fill_byte(0xFF)
        synchronize()
        graph.launch(stream)
        stream.synchronize()
        assert np.array_equal(out["dev"].numpy().view(np.uint16), ref.view(np.uint16)), rep
    assert min(tails) > 0, "every replay must include thin tails"
