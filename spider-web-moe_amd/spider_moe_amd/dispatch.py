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


@torch.no_grad()
def dispatch_expert_ffn(messages, top_indices, top_weights, *, w_up, b_up, w_down, b_down,
                        num_experts, expert_fn=None):
    """dispatch.py:145-185: dispatch -> local expert FFN -> combine.

    Without expert_fn the FFN (Linear + bias, erf GELU, Linear + bias) is
    sparse_expert_delta on the grouped GEMM kernels.  With expert_fn, the
    plan comes from the GPU plan kernels and, for each non-empty expert in
    ascending order, expert_fn(expert_id, tokens) runs on that expert's
    packed token rows (dispatch_tokens, :118-124); its outputs are stacked
    in plan order and the weighted combine (combine_tokens, :127-134: each
    output times its routing weight, added per token in ascending expert
    order) runs as one kernel (smoe_combine_rows).  messages [B,T,H] or
    [N,H]; returns delta in messages' shape and dtype."""
    if expert_fn is None:
        m3 = messages if messages.ndim == 3 else messages.unsqueeze(1)
        k = top_indices.shape[-1]
        d = sparse_expert_delta(m3, top_indices.reshape(m3.shape[0], m3.shape[1], k),
                                top_weights.reshape(m3.shape[0], m3.shape[1], k), w_up, b_up,
                                w_down, b_down, num_experts=num_experts, top_k=k)
        return d.view_as(messages)
    dev = nat.require_gpu(messages, top_indices, top_weights)
    if messages.dtype not in (torch.float32, torch.bfloat16):
        raise TypeError("messages must be float32 or bfloat16")
    h = messages.shape[-1]
    flat = messages.reshape(-1, h)
    plan = build_dispatch_plan(top_indices.reshape(flat.shape[0], -1),
                               top_weights.reshape(flat.shape[0], -1), num_experts=num_experts)
    rows = plan.rows.numel()
    y = torch.empty(max(rows, 1), h, dtype=messages.dtype, device=dev)
    off = 0
    for asg in plan.assignments:
        out = expert_fn(asg.expert_id, flat.index_select(0, asg.token_index))
        n = asg.token_index.numel()
        if out.shape != (n, h):
            raise ValueError(f"expert_fn returned {tuple(out.shape)} for {n} tokens; "
                             f"expected ({n}, {h})")
        y[off:off + n] = out.to(messages.dtype)
        off += n
    dt = nat.dtype_code(messages.dtype)
    delta = torch.empty(flat.shape[0], h, dtype=messages.dtype, device=dev)
    k = plan.token_rows.shape[-1]
    nat.check(nat.lib().smoe_combine_rows(y.data_ptr(), dt, plan.row_weights.data_ptr(),
                                          plan.token_rows.data_ptr(), flat.shape[0], k, h,
                                          delta.data_ptr(), dt, nat.stream_of(dev)),
              "smoe_combine_rows")
    plan.hidden = h
    return delta.view_as(messages)
