"""The explicit dispatch plan (spider_infer/forge/ep/dispatch.py:31-189) on
the GPU: build_dispatch_plan returns the reference's DispatchPlan /
ExpertAssignment structures, computed by smoe_dispatch_plan (slot merge +
stable count / scan / scatter); dispatch_expert_ffn is sparse_expert_delta.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _native as nat
from .sparse_experts import sparse_expert_delta


@dataclass
class ExpertAssignment:
    expert_id: int
    token_index: torch.Tensor  # [n] int64 flat positions
    weights: torch.Tensor      # [n] routing weights for this expert


@dataclass
class DispatchPlan:
    batch: int
    seq: int
    hidden: int
    top_k: int
    num_experts: int
    assignments: list = field(default_factory=list)
    local_expert_ids: list = field(default_factory=list)
    # flat device tensors of the plan (rows in (expert, token) order)
    counts: torch.Tensor | None = None
    offsets: torch.Tensor | None = None
    rows: torch.Tensor | None = None
    row_weights: torch.Tensor | None = None
    token_rows: torch.Tensor | None = None

    def tokens_for(self, expert_id: int):
        for a in self.assignments:
            if a.expert_id == expert_id:
                return a
        return None


@torch.no_grad()
def plan_tensors(top_indices: torch.Tensor, top_weights: torch.Tensor, num_experts: int):
    """Device plan: counts [E], offsets [E+1], rows [N*K], row_w [N*K],
    tok_row [N,K] (see include/smoe.h smoe_dispatch_plan)."""
    dev = nat.require_gpu(top_indices, top_weights)
    k = top_indices.shape[-1]
    idx = top_indices.reshape(-1, k).to(torch.int32).contiguous()
    w = top_weights.reshape(-1, k).to(torch.float32).contiguous()
    n = idx.shape[0]
    counts = torch.empty(num_experts, dtype=torch.int32, device=dev)
    offsets = torch.empty(num_experts + 1, dtype=torch.int32, device=dev)
    rows = torch.empty(max(n * k, 1), dtype=torch.int32, device=dev)
    roww = torch.empty(max(n * k, 1), dtype=torch.float32, device=dev)
    tokrow = torch.empty(max(n * k, 1), dtype=torch.int32, device=dev)
    lib = nat.lib()
    need = lib.smoe_dispatch_workspace_bytes(n, k, num_experts)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    nat.check(lib.smoe_dispatch_plan(idx.data_ptr(), w.data_ptr(), n, k, num_experts,
                                     counts.data_ptr(), offsets.data_ptr(), rows.data_ptr(),
                                     roww.data_ptr(), tokrow.data_ptr(), ws.data_ptr(), need,
                                     nat.stream_of(dev)),
              "smoe_dispatch_plan")
    return counts, offsets, rows, roww, tokrow[: n * k].view(n, k)


def build_dispatch_plan(top_indices, top_weights, *, num_experts: int, local_only: bool = True):
    """dispatch.py:56-115: top_indices / top_weights [B,T,K] or [N,K]."""
    if top_indices.ndim == 3:
        b, t, k = top_indices.shape
    elif top_indices.ndim == 2:
        (n, k), t = top_indices.shape, 1
        b = n
    else:
        raise ValueError("top_indices must be [B,T,K] or [N,K]")
    counts, offsets, rows, roww, tokrow = plan_tensors(top_indices, top_weights, num_experts)
    off = offsets.cpu().tolist()
    assignments = []
    for e in range(num_experts):
        if off[e + 1] > off[e]:
            assignments.append(ExpertAssignment(expert_id=e,
                                                token_index=rows[off[e]:off[e + 1]].long(),
                                                weights=roww[off[e]:off[e + 1]].clone()))
    return DispatchPlan(batch=b, seq=t, hidden=0, top_k=k, num_experts=num_experts,
                        assignments=assignments, local_expert_ids=list(range(num_experts)),
                        counts=counts, offsets=offsets, rows=rows[: off[-1]], row_weights=roww[: off[-1]],
                        token_rows=tokrow)


def dispatch_expert_ffn(messages, top_indices, top_weights, *, w_up, b_up, w_down, b_down,
                        num_experts, expert_fn=None):
    """dispatch.py:145-185 (the expert_fn callback form is not provided)."""
    if expert_fn is not None:
        raise NotImplementedError("expert_fn callbacks are not supported; the FFN runs in HIP")
    return sparse_expert_delta(messages, top_indices, top_weights, w_up, b_up, w_down, b_down,
                               num_experts=num_experts, top_k=top_indices.shape[-1])
