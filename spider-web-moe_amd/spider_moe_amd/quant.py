"""Expert weight formats (host-side packing; runs once, not per call).

int4: spider_moe/quant.py:76-143 — same function names, argument meaning and
bytes: symmetric per-group along the last dim, scale = max(amax, 1e-8) / 7,
q = clamp(round_half_even(w / scale), -8, 7), element 2i in the low nibble.
``scale_dtype=torch.float16`` stores the (identical) scales as fp16 — the
layout of the int4 decode/prefill configuration; the packed bytes do not
change.

fp8: per-output-channel e4m3 — scale = max(amax_K / 448, 1e-12) and
codes = (w / scale).to(float8_e4m3fn), as quantize_fp8_with_scale_tensor
(quant.py:146-158) with a [.., N] scale; dequant = code * scale
(quant.py:161-169).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

FP8_E4M3_MAX = 448.0


@dataclass
class Int4Tensor:
    """Packed INT4 weights with per-group scales (quant.py:76-86)."""

    packed: torch.Tensor
    scales: torch.Tensor
    shape: tuple
    group_size: int

    def dequantize(self, dtype: torch.dtype | None = None) -> torch.Tensor:
        return dequantize_int4(self.packed, self.scales, self.shape, self.group_size, dtype=dtype)


def quantize_int4(weight: torch.Tensor, group_size: int = 64,
                  scale_dtype: torch.dtype = torch.float32) -> Int4Tensor:
    """quant.py:89-117 (plus an optional fp16 scale storage)."""
    if weight.ndim < 1:
        raise ValueError("weight must be at least 1D")
    *lead, n = weight.shape
    if n % 2 != 0:
        raise ValueError("last dimension must be even for INT4 packing")
    if group_size <= 0 or n % group_size != 0:
        group_size = n
    g = group_size
    w = weight.detach().float().reshape(-1, n // g, g)
    scales = w.abs().amax(dim=-1).clamp_min(1e-8) / 7.0
    q = torch.round(w / scales.unsqueeze(-1)).clamp(-8, 7).to(torch.int8).reshape(-1, n)
    lo = (q[:, 0::2] & 0x0F).to(torch.uint8)
    hi = (q[:, 1::2] & 0x0F).to(torch.uint8)
    packed = (lo | (hi << 4)).reshape(*lead, n // 2).contiguous()
    return Int4Tensor(packed=packed, scales=scales.to(scale_dtype).reshape(*lead, n // g).contiguous(),
                      shape=tuple(weight.shape), group_size=g)


def dequantize_int4(packed, scales, shape, group_size, dtype=None):
    """quant.py:120-143."""
    *lead, half = packed.shape
    n = half * 2
    flat = packed.reshape(-1, half)
    lo = (flat & 0x0F).to(torch.int8)
    hi = ((flat >> 4) & 0x0F).to(torch.int8)
    lo = torch.where(lo >= 8, lo - 16, lo)
    hi = torch.where(hi >= 8, hi - 16, hi)
    q = torch.empty(flat.shape[0], n, device=packed.device, dtype=torch.int8)
    q[:, 0::2] = lo
    q[:, 1::2] = hi
    g = group_size
    w = (q.view(q.shape[0], n // g, g).float() * scales.float().reshape(q.shape[0], n // g, 1))
    w = w.view(*lead, n)
    if dtype is not None:
        w = w.to(dtype)
    return w.view(shape)


def _quantize_fp8_device(weight: torch.Tensor, per_row: bool):
    """smoe_quantize_fp8_tensor: the reference's scale and cast with IEEE
    divisions, the bits torch computes on the CPU (torch's GPU kernels
    divide by a reciprocal: an ulp off in the scale and, rarely, one code
    step off)."""
    from . import _native as nat
    w = weight.detach()
    if w.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        w = w.float()
    w = w.contiguous()
    k = w.shape[-1]
    rows = w.numel() // k if k else 0
    kp = -(-k // 4) * 4
    codes = torch.empty(rows, kp, dtype=torch.uint8, device=w.device)
    scale = torch.empty(rows if per_row else 1, dtype=torch.float32, device=w.device)
    lib = nat.lib()
    wsp = None if per_row else torch.empty(lib.smoe_quantize_fp8_workspace_bytes(),
                                           dtype=torch.uint8, device=w.device)
    code = nat.F16 if w.dtype == torch.float16 else nat.dtype_code(w.dtype)
    with torch.cuda.device(w.device):
        nat.check(lib.smoe_quantize_fp8_tensor(w.data_ptr(), code, rows, k, kp, int(per_row),
                                               codes.data_ptr(), scale.data_ptr(), nat.ptr(wsp),
                                               0 if wsp is None else wsp.numel(),
                                               nat.stream_of(w.device)),
                  "smoe_quantize_fp8_tensor")
    if kp != k:
        codes = codes[:, :k].contiguous()
    return codes.view(torch.float8_e4m3fn).view(w.shape), scale


def quantize_fp8_per_channel(weight: torch.Tensor):
    """[..., N, K] -> (float8_e4m3fn codes [..., N, K], float32 scale [..., N]).
    On a GPU: the HIP quantizer (same bits as the CPU formula)."""
    if weight.is_cuda and weight.numel():
        codes, scale = _quantize_fp8_device(weight, per_row=True)
        return codes, scale.view(weight.shape[:-1])
    w = weight.detach().float()
    scale = (w.abs().amax(dim=-1) / FP8_E4M3_MAX).clamp_min(1e-12)
    codes = (w / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    return codes.contiguous(), scale.contiguous()


def dequantize_fp8_per_channel(codes: torch.Tensor, scale: torch.Tensor,
                               dtype: torch.dtype = torch.float32) -> torch.Tensor:
    return (codes.float() * scale.float().unsqueeze(-1)).to(dtype)


def quantize_fp8_per_tensor(weight: torch.Tensor):
    """One scale for the whole tensor, the format of the reference's
    quantize_fp8 / compute_fp8_scale (quant.py:30-56): scale = max(amax / 448,
    1e-12) (fp32, a 0-dim tensor), codes = (w.float() / scale) cast to
    float8_e4m3fn (round to nearest even).  On a GPU: the HIP quantizer
    (same bits as the CPU formula)."""
    if weight.is_cuda and weight.numel():
        codes, scale = _quantize_fp8_device(weight, per_row=False)
        return codes, scale.reshape(())
    w = weight.detach().float()
    scale = (w.abs().amax() / FP8_E4M3_MAX).clamp_min(1e-12)
    return (w / scale).to(torch.float8_e4m3fn).contiguous(), scale


# ------------------------------------------------------ SwiGLU layout ----
SWIGLU_BLOCK = 32


def interleave_gate_up(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """[..., U, X] gate and up -> [..., 2U, X] with 32-row blocks alternating
    gate / up: rows [64j, 64j+32) = gate[32j:32j+32], rows [64j+32, 64j+64) =
    up[32j:32j+32] (the order the up-GEMM epilogue pairs them in)."""
    *lead, u, x = gate.shape
    if u % SWIGLU_BLOCK:
        raise ValueError("SwiGLU hidden size must be a multiple of 32")
    gb = gate.reshape(*lead, u // SWIGLU_BLOCK, SWIGLU_BLOCK, x)
    ub = up.reshape(*lead, u // SWIGLU_BLOCK, SWIGLU_BLOCK, x)
    return torch.stack([gb, ub], dim=-3).reshape(*lead, 2 * u, x).contiguous()


def interleave_gate_up_rows(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """Same interleave for per-row vectors [..., U] (fp8 scales)."""
    return interleave_gate_up(gate.unsqueeze(-1), up.unsqueeze(-1)).squeeze(-1)
