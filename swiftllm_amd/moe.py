"""MoE top-k routing and expert-contiguous dispatch on the GPU.

Mirrors the steps MoeMlp::forward names
(crates/swiftllm-models/src/layers/mlp.rs:207-252: router logits, top-k,
route tokens to experts, combine), which the reference leaves as a zero stub.
Ranking conventions follow crates/swiftllm-core/src/sampling/mod.rs:366-385.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import _lib
from ._hip import DeviceArray, Stream
from .paged_attention import check_status


def moe_route(logits: DeviceArray, top_k: int, expert_ids: DeviceArray, weights: DeviceArray,
              stream: Optional[Stream] = None) -> None:
    """logits fp32 [T, E] -> expert_ids int32 [T, K], weights fp32 [T, K]."""
    T, E = logits.shape
    check_status(_lib.lib().swiftllm_hip_moe_route(
        logits.ptr, T, E, top_k, expert_ids.ptr, weights.ptr,
        stream.handle if stream else None))


def moe_dispatch_workspace_size(num_tokens: int, num_experts: int, top_k: int) -> int:
    n = _lib.lib().swiftllm_hip_moe_dispatch_workspace_size(num_tokens, num_experts, top_k)
    if n == 0:
        check_status(_lib.lib().swiftllm_hip_last_error() or -4)
    return int(n)


@dataclass
class DispatchBuffers:
    counts: DeviceArray        # int32 [E]
    offsets: DeviceArray       # int32 [E + 1]
    x_perm: Optional[DeviceArray]  # fp16 [T*K, hidden]
    inverse: DeviceArray       # int32 [T, K]
    sorted_token_ids: DeviceArray  # int32 [T*K]
    workspace: DeviceArray

    @classmethod
    def allocate(cls, num_tokens: int, num_experts: int, top_k: int, hidden: int,
                 with_rows: bool = True) -> "DispatchBuffers":
        n = moe_dispatch_workspace_size(num_tokens, num_experts, top_k)
        ws = DeviceArray((max(n, 4) + 3) // 4, np.uint32)   # plain scratch
        return cls(
            counts=DeviceArray((num_experts,), np.int32),
            offsets=DeviceArray((num_experts + 1,), np.int32),
            x_perm=DeviceArray((num_tokens * top_k, hidden), np.float16) if with_rows else None,
            inverse=DeviceArray((num_tokens, top_k), np.int32),
            sorted_token_ids=DeviceArray((max(num_tokens * top_k, 1),), np.int32),
            workspace=ws,
        )


def moe_dispatch(expert_ids: DeviceArray, x: Optional[DeviceArray], num_experts: int,
                 out: DispatchBuffers, stream: Optional[Stream] = None) -> None:
    T, K = expert_ids.shape
    hidden = x.shape[1] if x is not None else 0
    check_status(_lib.lib().swiftllm_hip_moe_dispatch(
        expert_ids.ptr, x.ptr if x is not None else None, T, K, num_experts, hidden,
        out.counts.ptr, out.offsets.ptr, out.x_perm.ptr if out.x_perm is not None else None,
        out.inverse.ptr, out.sorted_token_ids.ptr, out.workspace.ptr, out.workspace.nbytes,
        stream.handle if stream else None))


def moe_route_dispatch(logits: DeviceArray, x: Optional[DeviceArray], top_k: int,
                       expert_ids: DeviceArray, weights: DeviceArray, out: DispatchBuffers,
                       stream: Optional[Stream] = None) -> None:
    """moe_route then moe_dispatch in one call: the routing runs inside the
    dispatch's ranking kernel."""
    T, E = logits.shape
    hidden = x.shape[1] if x is not None else 0
    check_status(_lib.lib().swiftllm_hip_moe_route_dispatch(
        logits.ptr, x.ptr if x is not None else None, T, top_k, E, hidden, expert_ids.ptr,
        weights.ptr, out.counts.ptr, out.offsets.ptr,
        out.x_perm.ptr if out.x_perm is not None else None, out.inverse.ptr,
        out.sorted_token_ids.ptr, out.workspace.ptr, out.workspace.nbytes,
        stream.handle if stream else None))


def moe_expert_gemm(a: DeviceArray, w: DeviceArray, w2: Optional[DeviceArray],
                    expert_offsets: DeviceArray, c: DeviceArray,
                    stream: Optional[Stream] = None) -> None:
    """Grouped expert GEMM over expert-contiguous rows: a fp16 [m_total, k],
    w (and w2) fp16 [E, n, k], c fp16 [m_total, n]; with w2 the SwiGLU
    product silu(a.w^T) * (a.w2^T)."""
    m_total, k = a.shape
    E, n, kw = w.shape
    if kw != k or c.shape != (m_total, n) or (w2 is not None and w2.shape != w.shape):
        raise ValueError(f"shapes a{a.shape} w{w.shape} c{c.shape}")
    check_status(_lib.lib().swiftllm_hip_moe_expert_gemm(
        a.ptr, w.ptr, w2.ptr if w2 is not None else None, expert_offsets.ptr, E, m_total, n, k,
        c.ptr, stream.handle if stream else None))


def moe_combine(y: DeviceArray, weights: DeviceArray, inverse: DeviceArray, out: DeviceArray,
                stream: Optional[Stream] = None) -> None:
    """out[t] = sum_k weights[t, k] * y[inverse[t, k]] (fp32, then fp16)."""
    T, K = inverse.shape
    rows, hidden = y.shape
    check_status(_lib.lib().swiftllm_hip_moe_combine(
        y.ptr, weights.ptr, inverse.ptr, T, K, hidden, rows, out.ptr,
        stream.handle if stream else None))


class MoeMlp:
    """MoeMlp::forward (mlp.rs:207-252) from router logits on: top-k
    routing, dispatch, the gated expert GEMM (GatedMlp, mlp.rs:118-160), the
    down-projection GEMM and the weighted combine. Expert weights are stacked
    fp16 device arrays: gate_proj and up_proj [E, I, hidden], down_proj
    [E, hidden, I]."""

    def __init__(self, num_experts: int, num_experts_per_tok: int, gate_proj: DeviceArray,
                 up_proj: DeviceArray, down_proj: DeviceArray):
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.gate_proj, self.up_proj, self.down_proj = gate_proj, up_proj, down_proj
        self.intermediate = gate_proj.shape[1]
        self._bufs = {}

    def buffers(self, T: int, hidden: int):
        key = (T, hidden)
        if key not in self._bufs:
            K, I = self.num_experts_per_tok, self.intermediate
            self._bufs[key] = dict(
                ids=DeviceArray((T, K), np.int32), weights=DeviceArray((T, K), np.float32),
                dispatch=DispatchBuffers.allocate(T, self.num_experts, K, hidden),
                h=DeviceArray((max(T * K, 1), I), np.float16),
                y=DeviceArray((max(T * K, 1), hidden), np.float16),
                out=DeviceArray((T, hidden), np.float16))
        return self._bufs[key]

    def forward(self, router_logits: DeviceArray, x: DeviceArray,
                stream: Optional[Stream] = None) -> DeviceArray:
        T, hidden = x.shape
        b = self.buffers(T, hidden)
        d = b["dispatch"]
        moe_route_dispatch(router_logits, x, self.num_experts_per_tok, b["ids"], b["weights"], d,
                           stream)
        if T > 0:
            moe_expert_gemm(d.x_perm, self.gate_proj, self.up_proj, d.offsets, b["h"], stream)
            moe_expert_gemm(b["h"], self.down_proj, None, d.offsets, b["y"], stream)
        moe_combine(b["y"], b["weights"], d.inverse, b["out"], stream)
        return b["out"]


class MoeRouting:
    """The routing half of MoeMlp (mlp.rs:209-221 fields num_experts,
    num_experts_per_tok): route(logits) then dispatch(x)."""

    def __init__(self, num_experts: int, num_experts_per_tok: int):
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok

    def forward(self, router_logits: DeviceArray, x: DeviceArray,
                stream: Optional[Stream] = None):
        T = router_logits.shape[0]
        K = self.num_experts_per_tok
        ids = DeviceArray((T, K), np.int32)
        w = DeviceArray((T, K), np.float32)
        bufs = DispatchBuffers.allocate(T, self.num_experts, K, x.shape[1])
        moe_route_dispatch(router_logits, x, K, ids, w, bufs, stream)
        return ids, w, bufs
