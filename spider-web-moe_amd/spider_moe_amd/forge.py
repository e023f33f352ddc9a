"""Forge surfaces (spider_infer/forge/*) on the block's HIP kernels.

The reference's kernel fabric exposes three of the block's operations with
its own call surface and slightly different semantics (forge/select,
forge/gemm, forge/ep).  Here they run on libsmoe.so:

  ForgeSelect.route    top-k on the logits, softmax over the k values
                       (forge/select/api.py:28-40) -> smoe_select_topk
  ForgeGEMM.linear / linear_fp8 / expert_ffn, fp8_linear /
  fp8_expert_ffn       (forge/gemm/api.py:34-74, fp8.py:22-78,
                       triton_kernels.py:65-123) -> smoe_linear; fp8
                       weights use the reference's per-tensor scale
                       (quantize_fp8), cached per weight version;
                       quantize_input -> smoe_quantize_fp8_tensor +
                       smoe_linear_fp8fp8 (e4m3 x e4m3 MFMA)
  ForgeEP.dispatch_plan / run_dispatched_ffn / combine
                       (forge/ep/api.py:46-104) -> the dispatch plan
                       kernels, sparse_expert_delta, or an expert_fn
                       callback per assignment with the weighted combine
                       on the GPU (dispatch.dispatch_expert_ffn)

One GPU: the cross-rank combine is the identity (no process group), as
the reference's combine_across_ranks is at world size 1.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from enum import Enum
from typing import Any, Callable

import torch

from . import _native as nat
from .dispatch import DispatchPlan, build_dispatch_plan, dispatch_expert_ffn
from .quant import quantize_fp8_per_tensor


class ForgeBackend(str, Enum):
    """forge/config.py:8-16; this build has one backend."""
    HIP = "hip"


@dataclass
class ForgeConfig:
    """The fields of forge/config.py:19-51 that these surfaces read."""
    gemm_fp8: bool = False
    ep_enabled: bool = True
    ep_async: bool = False
    select_top_k: int = 2
    select_top_dobu: int = 4

    def to_dict(self) -> dict:
        return {"gemm_fp8": self.gemm_fp8, "ep": self.ep_enabled, "ep_async": self.ep_async,
                "select_top_k": self.select_top_k, "select_top_dobu": self.select_top_dobu,
                "backend": ForgeBackend.HIP.value}


# ---------------------------------------------------------------- select ----
class ForgeSelect:
    """Router selection with explicit top_k (compute) vs top_dobu (the Dobu
    residency budget, reported, not used as k)."""

    def __init__(self, config: ForgeConfig | None = None):
        self.config = config or ForgeConfig()
        self.calls = 0

    @torch.no_grad()
    def route(self, logits: torch.Tensor, *, top_k: int | None = None):
        """logits [..., E] -> (top_weights, top_indices) [..., k]: top-k on
        the logits, softmax over the k values; weights in the logits'
        dtype (computed in fp32), indices int64 as torch.topk returns."""
        self.calls += 1
        e = logits.shape[-1]
        k = int(top_k if top_k is not None else self.config.select_top_k)
        k = max(1, min(k, e))
        return select_topk(logits, k, nat.SMOE_SELECT_TOPK_SOFTMAX)

    def top_dobu_budget(self) -> int:
        return int(self.config.select_top_dobu)

    def stats(self) -> dict[str, Any]:
        return {"pillar": "select", "impl": "hip_select_topk", "backend": ForgeBackend.HIP.value,
                "calls": self.calls, "top_k": self.config.select_top_k,
                "top_dobu": self.config.select_top_dobu}


def select_topk(logits: torch.Tensor, k: int, mode: int):
    """smoe_select_topk over the last dimension (E <= 64)."""
    dev = nat.require_gpu(logits)
    e = logits.shape[-1]
    lead = logits.shape[:-1]
    x = logits.reshape(-1, e).to(torch.float32).contiguous()
    n = x.shape[0]
    w = torch.empty(n, k, dtype=torch.float32, device=dev)
    idx = torch.empty(n, k, dtype=torch.int32, device=dev)
    nat.check(nat.lib().smoe_select_topk(x.data_ptr(), n, e, k, mode, w.data_ptr(), idx.data_ptr(),
                                         nat.stream_of(dev)), "smoe_select_topk")
    out_dtype = logits.dtype if logits.dtype.is_floating_point else torch.float32
    return w.view(*lead, k).to(out_dtype), idx.view(*lead, k).long()


# ------------------------------------------------------------------ gemm ----
_ACT = {None: 0, "gelu": 1}


def _linear(x: torch.Tensor, w: torch.Tensor, w_format: int, scale, bias, act, out_dtype):
    """smoe_linear: x [..., K] . w^T (+ bias, act) -> [..., N_out]."""
    dev = nat.require_gpu(x, w)
    k = x.shape[-1]
    lead = x.shape[:-1]
    xa = x.reshape(-1, k).to(torch.float32 if w_format == nat.F32 else torch.bfloat16).contiguous()
    n = xa.shape[0]
    n_out = w.shape[0]
    out = torch.empty(n, n_out, dtype=out_dtype, device=dev)
    b = None if bias is None else bias.detach().float().contiguous()
    nat.check(nat.lib().smoe_linear(xa.data_ptr(), n, k, w.data_ptr(), w_format, nat.ptr(scale),
                                    nat.ptr(b), n_out, _ACT[act], out.data_ptr(),
                                    nat.dtype_code(out_dtype), nat.stream_of(dev)), "smoe_linear")
    return out.view(*lead, n_out)


class _Fp8Cache:
    """Per-tensor fp8 codes of a weight, re-quantized when the weight
    changes (the reference quantizes on every call, fp8.py:46), in the
    forms the kernels read: the codes [N_out, K] with the scale repeated per
    channel (weight-only GEMM), the codes zero-padded to K % 256 == 0 with
    the scale as one f32 (fp8 x fp8 GEMM), and the dequantized f32 weight
    codes * scale (fp32 inputs, which the reference multiplies in fp32)."""

    def __init__(self):
        self._c: dict = {}

    def _entry(self, w: torch.Tensor) -> dict:
        key = (w.data_ptr(), w._version, tuple(w.shape), w.dtype)
        hit = self._c.get(id(w))
        if hit is not None and hit[0] == key:
            return hit[1]
        codes, scale = quantize_fp8_per_tensor(w)
        ent = {"codes": codes.view(torch.uint8), "scale": scale.reshape(1).to(w.device)}
        self._c[id(w)] = (key, ent)
        return ent

    def get(self, w: torch.Tensor):
        ent = self._entry(w)
        if "scale_vec" not in ent:
            ent["scale_vec"] = ent["scale"].expand(w.shape[0]).contiguous()
        return ent["codes"], ent["scale_vec"]

    def get_padded(self, w: torch.Tensor):
        ent = self._entry(w)
        if "padded" not in ent:
            k = w.shape[1]
            kp = -(-k // 256) * 256
            pad = torch.zeros(w.shape[0], kp, dtype=torch.uint8, device=w.device)
            pad[:, :k] = ent["codes"]
            ent["padded"] = pad
        return ent["padded"], ent["scale"]

    def get_dequant(self, w: torch.Tensor):
        ent = self._entry(w)
        if "deq" not in ent:
            ent["deq"] = (ent["codes"].view(torch.float8_e4m3fn).float() * ent["scale"]).contiguous()
        return ent["deq"]


def quantize_fp8_input(x: torch.Tensor, k_pad: int):
    """Per-tensor e4m3 codes of x [..., K] on the device (smoe_quantize_fp8_tensor:
    quant.py:30-56's scale and round-to-nearest-even cast) as [rows, k_pad]
    u8 with zero codes past K, and the scale (f32 [1])."""
    dev = nat.require_gpu(x)
    k = x.shape[-1]
    xa = x.reshape(-1, k)
    if xa.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        xa = xa.float()
    xa = xa.contiguous()
    rows = xa.shape[0]
    codes = torch.empty(rows, k_pad, dtype=torch.uint8, device=dev)
    scale = torch.empty(1, dtype=torch.float32, device=dev)
    lib = nat.lib()
    ws = torch.empty(lib.smoe_quantize_fp8_workspace_bytes(), dtype=torch.uint8, device=dev)
    code = nat.F16 if xa.dtype == torch.float16 else nat.dtype_code(xa.dtype)
    nat.check(lib.smoe_quantize_fp8_tensor(xa.data_ptr(), code, rows, k, k_pad, 0,
                                           codes.data_ptr(), scale.data_ptr(), ws.data_ptr(),
                                           ws.numel(), nat.stream_of(dev)),
              "smoe_quantize_fp8_tensor")
    return codes, scale


class ForgeGEMM:
    """ForgeGEMM (forge/gemm/api.py:22-87) on the block's GEMM kernels.

    linear: x . w^T + b in fp32 on the values of x / w (bf16 inputs run
    the bf16 MFMA path with fp32 accumulation, f32 inputs the fp32 path),
    result in x's dtype.  With config.gemm_fp8 (or linear_fp8) the weight is
    quantized to e4m3 with one per-tensor scale (quantize_fp8): bf16 / f16
    inputs run the GEMM on the codes (activations read as bf16, the scale
    in the epilogue), f32 inputs the fp32 GEMM on the dequantized weight
    (the reference's fp32 compute dtype, fp8.py:41-54).  quantize_input:
    x is quantized per tensor too (smoe_quantize_fp8_tensor) and the GEMM
    multiplies e4m3 by e4m3 (smoe_linear_fp8fp8, the f8f6f4 MFMA), both
    scales applied in f32.  expert_ffn: linear, GELU (erf), linear."""

    def __init__(self, config: ForgeConfig | None = None):
        self.config = config or ForgeConfig()
        self.calls = 0
        self._fp8 = _Fp8Cache()
        self.last_fp8_backend = "not_run"

    def _run(self, x, w, bias, act, fp8, quantize_input=False):
        """fp8: e4m3 weight codes; else fp32 when x or w is fp32 (exact
        products of their values), bf16 x bf16 otherwise."""
        if fp8 and quantize_input:
            return self._run_fp8fp8(x, w, bias, act)
        if fp8 and x.dtype == torch.float32:
            wt, fmt, scale = self._fp8.get_dequant(w), nat.F32, None
            self.last_fp8_backend = "hip_fp8_weight_dequant_f32"
        elif fp8:
            wt, scale = self._fp8.get(w)
            fmt = nat.FP8_E4M3
            self.last_fp8_backend = "hip_fp8_weight_bf16_mfma"
        elif x.dtype == torch.float32 or w.dtype == torch.float32:
            wt, fmt, scale = w.detach().float().contiguous(), nat.F32, None
        else:
            wt, fmt, scale = w.detach().to(torch.bfloat16).contiguous(), nat.BF16, None
        out_dtype = torch.float32 if (act is None or fmt == nat.F32) else torch.bfloat16
        return _linear(x, wt, fmt, scale, bias, act, out_dtype)

    def _run_fp8fp8(self, x, w, bias, act):
        dev = nat.require_gpu(x, w)
        wq, ws = self._fp8.get_padded(w)
        k_pad = wq.shape[1]
        xq, xs = quantize_fp8_input(x, k_pad)
        n, n_out = xq.shape[0], wq.shape[0]
        out_dtype = torch.bfloat16 if (act is not None and x.dtype != torch.float32) else torch.float32
        out = torch.empty(n, n_out, dtype=out_dtype, device=dev)
        b = None if bias is None else bias.detach().float().contiguous()
        nat.check(nat.lib().smoe_linear_fp8fp8(xq.data_ptr(), xs.data_ptr(), n, k_pad, wq.data_ptr(),
                                               ws.data_ptr(), nat.ptr(b), n_out, _ACT[act],
                                               out.data_ptr(), nat.dtype_code(out_dtype),
                                               nat.stream_of(dev)), "smoe_linear_fp8fp8")
        self.last_fp8_backend = "hip_fp8xfp8_mfma_f8f6f4"
        return out.view(*x.shape[:-1], n_out)

    @torch.no_grad()
    def linear(self, x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None):
        self.calls += 1
        return self._run(x, weight, bias, None, self.config.gemm_fp8).to(x.dtype)

    @torch.no_grad()
    def linear_fp8(self, x, weight, bias=None, *, quantize_input: bool = False):
        """Explicit fp8 path regardless of config.gemm_fp8 (fp8.py:22-62)."""
        self.calls += 1
        return self._run(x, weight, bias, None, True, quantize_input).to(x.dtype)

    @torch.no_grad()
    def expert_ffn(self, x, w_up, b_up, w_down, b_down):
        self.calls += 1
        fp8 = self.config.gemm_fp8
        h = self._run(x, w_up, b_up, "gelu", fp8)
        return self._run(h.to(x.dtype), w_down, b_down, None, fp8).to(x.dtype)

    @torch.no_grad()
    def fp8_expert_ffn(self, x, w_up, b_up, w_down, b_down, *, quantize_input: bool = False):
        """fp8.py:65-76: the up projection (input quantized when asked) with
        its GELU, then the down projection on fp8 weights only."""
        self.calls += 1
        h = self._run(x, w_up, b_up, "gelu", True, quantize_input)
        return self._run(h.to(x.dtype), w_down, b_down, None, True).to(x.dtype)

    def stats(self) -> dict[str, Any]:
        return {"pillar": "gemm", "impl": "hip_grouped_gemm", "backend": ForgeBackend.HIP.value,
                "calls": self.calls, "fp8": self.config.gemm_fp8,
                "last_fp8_kernel": self.last_fp8_backend}


_FP8_GEMM = None


def _fp8_gemm() -> "ForgeGEMM":
    global _FP8_GEMM
    if _FP8_GEMM is None:
        _FP8_GEMM = ForgeGEMM(ForgeConfig(gemm_fp8=True))
    return _FP8_GEMM


def fp8_linear(x, weight, bias=None, *, quantize_input: bool = False, compute_dtype=None):
    """forge/gemm/fp8.py:22-62 on the HIP kernels: per-tensor e4m3 weights
    (and, with quantize_input, activations); F.linear's shape, result in
    x's dtype.  compute_dtype is accepted for the reference's signature:
    the kernels accumulate in f32 whatever it says."""
    return _fp8_gemm().linear_fp8(x, weight, bias, quantize_input=quantize_input)


def fp8_expert_ffn(x, w_up, b_up, w_down, b_down, *, quantize_input: bool = False):
    """forge/gemm/fp8.py:65-76 on the HIP kernels."""
    return _fp8_gemm().fp8_expert_ffn(x, w_up, b_up, w_down, b_down, quantize_input=quantize_input)


def get_last_fp8_gemm_backend():
    """(kernel, error) of the last fp8 call (fp8.py:79-80); errors raise
    here instead of falling back."""
    return _fp8_gemm().last_fp8_backend, None


# -------------------------------------------------------------------- ep ----
class ForgeEP:
    """Token dispatch + combine (forge/ep/api.py:21-117) at world size 1."""

    def __init__(self, config: ForgeConfig | None = None):
        self.config = config or ForgeConfig()
        self.calls = 0

    def enabled(self) -> bool:
        return False  # one GPU: no expert-parallel group

    def rank_world(self) -> tuple[int, int]:
        return 0, 1

    def owns(self, expert_id: int) -> bool:
        return True  # expert_id % 1 == 0 (expert_parallel.py:29)

    def combine(self, delta: torch.Tensor) -> torch.Tensor:
        self.calls += 1
        return delta

    def dispatch_meta(self, top_indices: torch.Tensor, num_experts: int) -> dict:
        self.calls += 1
        plan = build_dispatch_plan(top_indices, torch.ones_like(top_indices, dtype=torch.float32),
                                   num_experts=num_experts, local_only=True)
        return {"rank": 0, "world": 1, "local_experts": plan.local_expert_ids,
                "assignments": len(plan.assignments), "top_indices_shape": list(top_indices.shape)}

    def dispatch_plan(self, top_indices, top_weights, num_experts: int) -> DispatchPlan:
        self.calls += 1
        return build_dispatch_plan(top_indices, top_weights, num_experts=num_experts,
                                   local_only=True)

    def run_dispatched_ffn(self, messages, top_indices, top_weights, *, w_up, b_up, w_down,
                           b_down, num_experts: int, expert_fn: Callable | None = None):
        self.calls += 1
        return dispatch_expert_ffn(messages, top_indices, top_weights, w_up=w_up, b_up=b_up,
                                   w_down=w_down, b_down=b_down, num_experts=num_experts,
                                   expert_fn=expert_fn)

    def stats(self) -> dict[str, Any]:
        return {"pillar": "ep", "impl": "hip_dispatch_plan", "backend": ForgeBackend.HIP.value,
                "calls": self.calls, "rank": 0, "world": 1, "async": self.config.ep_async}


# --------------------------------------------------------------- runtime ----
class ForgeRuntime:
    """The object init_forge returns (forge/registry.py:20-56): the pillars
    this build provides."""

    def __init__(self, config: ForgeConfig | None = None):
        self.config = config or ForgeConfig()
        self.select = ForgeSelect(self.config)
        self.gemm = ForgeGEMM(self.config)
        self.ep = ForgeEP(self.config)

    def stats(self) -> dict[str, Any]:
        return {"config": self.config.to_dict(), "select": self.select.stats(),
                "gemm": self.gemm.stats(), "ep": self.ep.stats()}


_RUNTIME: ForgeRuntime | None = None


def init_forge(config: ForgeConfig | None = None) -> ForgeRuntime:
    """forge/registry.py:58-88."""
    global _RUNTIME
    _RUNTIME = ForgeRuntime(config)
    return _RUNTIME


def get_forge() -> ForgeRuntime:
    """forge/registry.py:91-95: the runtime, created with defaults on first use."""
    return _RUNTIME if _RUNTIME is not None else init_forge()


__all__ = ["ForgeBackend", "ForgeConfig", "ForgeSelect", "ForgeGEMM", "ForgeEP", "ForgeRuntime",
           "init_forge", "get_forge", "select_topk", "fp8_linear", "fp8_expert_ffn",
           "get_last_fp8_gemm_backend", "quantize_fp8_input"]
