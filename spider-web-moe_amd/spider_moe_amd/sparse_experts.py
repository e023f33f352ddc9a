"""sparse_expert_delta with the reference signature (spider_moe/sparse_experts.py:11-68),
computed by libsmoe.so: slot merge -> stable dispatch plan -> grouped up
GEMM + GELU -> grouped down GEMM (+ bias, x routing weight) -> per-token
combine in ascending expert order.

Duplicate expert ids across slots add their weights; a token whose merged
weight is <= 0 is dropped for that expert (sparse_experts.py:52-56); ids
outside [0, E) match no expert.  Weights may be float32 or bfloat16
(messages are cast to bfloat16 for bf16 weights, the MFMA path).

With expert parallelism active (torch.distributed world > 1) the reference
computes its local experts and SUM-all-reduces; this single-GPU module
computes every expert on every rank, which yields the same delta.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native as nat


def _experts_desc(w_up, b_up, w_down, b_down, act=nat.ACT_GELU):
    e, u, h = w_up.shape
    ex = nat.SmoeExperts()
    ex.format = nat.dtype_code(w_up.dtype)
    ex.act = act
    ex.E, ex.H, ex.U = e, h, u
    keep = [w_up.contiguous(), w_down.to(w_up.dtype).contiguous()]
    ex.w_up, ex.w_down = keep[0].data_ptr(), keep[1].data_ptr()
    for name, b in (("b_up", b_up), ("b_down", b_down)):
        if b is not None:
            bb = b.detach().float().contiguous()
            keep.append(bb)
            setattr(ex, name, bb.data_ptr())
    return ex, keep


@torch.no_grad()
def sparse_expert_delta(
    messages: torch.Tensor,
    top_indices: torch.Tensor,
    top_weights: torch.Tensor,
    w_up: torch.Tensor,
    b_up: torch.Tensor,
    w_down: torch.Tensor,
    b_down: torch.Tensor,
    num_experts: int,
    top_k: int,
    expert_parallel: bool = True,
) -> torch.Tensor:
    """messages [B,T,H]; top_indices / top_weights [B,T,K]; w_up [E,U,H];
    b_up [E,U]; w_down [E,H,U]; b_down [E,H] -> delta [B,T,H] (messages.dtype)."""
    dev = nat.require_gpu(messages, top_indices, top_weights, w_up, b_up, w_down, b_down)
    b, t, width = messages.shape
    if w_up.shape[0] != num_experts or top_indices.shape[-1] != top_k:
        raise ValueError("num_experts / top_k do not match the tensors")
    n = b * t
    ex, keep = _experts_desc(w_up, b_up, w_down, b_down)
    ffn_dtype = torch.float32 if ex.format == nat.F32 else torch.bfloat16
    msg = messages.reshape(n, width).to(ffn_dtype).contiguous()
    idx = top_indices.reshape(n, top_k).to(torch.int32).contiguous()
    wts = top_weights.reshape(n, top_k).to(torch.float32).contiguous()
    out_dtype = messages.dtype if messages.dtype in (torch.float32, torch.bfloat16) else torch.float32
    delta = torch.empty(n, width, dtype=out_dtype, device=dev)
    lib = nat.lib()
    need = lib.smoe_expert_delta_workspace_bytes(ctypes.byref(ex), n, top_k)
    if need == 0:
        raise RuntimeError(f"smoe_expert_delta: unsupported expert shapes ({lib.smoe_last_error().decode()})")
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    nat.check(lib.smoe_expert_delta(ctypes.byref(ex), msg.data_ptr(), idx.data_ptr(), wts.data_ptr(),
                                    n, top_k, delta.data_ptr(), nat.dtype_code(out_dtype),
                                    ws.data_ptr(), need, nat.stream_of(dev)),
              "smoe_expert_delta")
    del keep
    return delta.view(b, t, width).to(messages.dtype)
