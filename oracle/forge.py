"""Oracle: the Forge surfaces on the CPU (TEST INFRASTRUCTURE ONLY).

Restatements, with torch on the CPU (the library the reference calls):

  select_route     forge/select/api.py:28-40: vals, idx = topk(logits, k);
                   weights = softmax(vals) (in the logits' dtype)
  fp8_linear       forge/gemm/fp8.py:22-62 with quant.py:30-69: per-tensor
                   scale = max(amax(|w|) / 448, 1e-12); codes =
                   (w.float() / scale) -> e4m3; w_deq = (codes.float() *
                   scale) in the compute dtype (fp16 for half / bf16 inputs,
                   else fp32); with quantize_input, x likewise; F.linear(
                   x_deq, w_deq, bias); the result in x's dtype
  fp8_expert_ffn   fp8.py:65-76: fp8_linear (quantize_input), GELU,
                   fp8_linear
  expert_ffn       fp8.py:65-75 / triton_kernels.py:113-123: linear, GELU
                   (erf), linear
  dispatch_ffn     forge/ep/dispatch.py:145-185: for each expert ascending
                   with a positive merged weight (oracle.plan), tokens =
                   messages[positions]; out = expert_fn(e, tokens);
                   delta.index_add_(0, positions, out * weights)

Pins (tests/test_oracle_native_forge.py): hand-computed known answers for the
selection; the per-tensor scale and codes against the closed form and the
e4m3 decode table of oracle/quant.py; quantize_input against a known answer
(values on the e4m3 grid pass unchanged), the scale-invariance of the codes
(x and 2^j x give the same codes, the scale times 2^j) and a planted
mistake (codes without the input scale); the dispatch combine against a
per-token loop over the dense merged weights.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import plan as plan_mod

FP8_E4M3_MAX = 448.0


def select_route(logits: torch.Tensor, k: int):
    vals, idx = torch.topk(logits, k=k, dim=-1)
    return F.softmax(vals, dim=-1), idx


def fp8_quantize_per_tensor(w: torch.Tensor):
    scale = (w.detach().float().abs().amax() / FP8_E4M3_MAX).clamp_min(1e-12)
    return (w.float() / scale).to(torch.float8_e4m3fn), scale


def fp8_linear(x: torch.Tensor, w: torch.Tensor, bias=None, *, quantize_input: bool = False):
    """fp8.py:22-62.  quantize_input: x is quantized per tensor as w is
    (fp8.py:49-51) and dequantized in the compute dtype."""
    compute = torch.float16 if x.dtype in (torch.float16, torch.bfloat16) else torch.float32
    codes, scale = fp8_quantize_per_tensor(w)
    w_deq = (codes.float() * scale).to(compute)
    if quantize_input:
        xc, xs = fp8_quantize_per_tensor(x)
        x_deq = (xc.float() * xs).to(compute)
    else:
        x_deq = x.to(compute)
    b = None if bias is None else bias.to(compute)
    return F.linear(x_deq, w_deq, b).to(x.dtype)


def fp8_expert_ffn(x, w_up, b_up, w_down, b_down, *, quantize_input: bool = False):
    """fp8.py:65-76: the up projection with the input quantized when asked,
    GELU (erf), the down projection on fp8 weights only."""
    h = F.gelu(fp8_linear(x, w_up, b_up, quantize_input=quantize_input))
    return fp8_linear(h, w_down, b_down)


def linear(x: torch.Tensor, w: torch.Tensor, bias=None):
    """triton_kernels.py:65-110: fp32 GEMM on the values, cast to x's dtype,
    then + bias."""
    out = (x.float() @ w.float().t()).to(x.dtype)
    return out if bias is None else out + bias.to(x.dtype)


def expert_ffn(x, w_up, b_up, w_down, b_down, fp8: bool):
    lin = fp8_linear if fp8 else linear
    h = F.gelu(lin(x, w_up, b_up))
    return lin(h, w_down, b_down)


def dispatch_ffn(messages: torch.Tensor, top_i: torch.Tensor, top_w: torch.Tensor,
                 num_experts: int, expert_fn):
    flat = messages.reshape(-1, messages.shape[-1])
    k = top_i.shape[-1]
    assignments, *_ = plan_mod.dispatch_plan(top_i.reshape(-1, k).numpy(),
                                             top_w.reshape(-1, k).float().numpy(), num_experts)
    delta = torch.zeros_like(flat)
    for eid, pos, wts in assignments:
        p = torch.from_numpy(pos)
        out = expert_fn(eid, flat.index_select(0, p))
        delta.index_add_(0, p, out * torch.from_numpy(wts).to(out.dtype).unsqueeze(-1))
    return delta.view_as(messages)
