"""ctypes binding of libsmoe.so (the gfx950 HIP kernels behind include/smoe.h).

torch is imported before the library is opened: PyTorch-ROCm ships its own
HIP runtime with soname libamdhip64.so.7, and libsmoe.so then binds to that
already-loaded runtime, so device pointers and streams are shared.  There is
no fallback: when the library is missing every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must precede loading libsmoe.so, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libsmoe.so")

# formats / activations / status codes (include/smoe.h)
F32, BF16, FP8_E4M3, INT4, F16 = 0, 1, 2, 3, 4
ACT_GELU, ACT_SWIGLU = 0, 1
SMOE_SELECT_ROUTER, SMOE_SELECT_TOPK_SOFTMAX = 0, 1
STATUS = {0: "ok", 1: "invalid argument", 2: "index out of range", 3: "capacity",
          -2: "unsupported dtype/format", 4: "HIP runtime error"}

_c_int, _c_float, _vp, _sz = ctypes.c_int, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t


class SmoeExperts(ctypes.Structure):
    _fields_ = [("format", _c_int), ("act", _c_int), ("E", _c_int), ("H", _c_int), ("U", _c_int),
                ("group_size", _c_int), ("scale_dtype", _c_int),
                ("w_up", _vp), ("w_gate", _vp), ("w_down", _vp), ("s_up", _vp), ("s_down", _vp),
                ("b_up", _vp), ("b_down", _vp), ("w_up_tiles", _vp), ("w_down_tiles", _vp)]


class SmoeBlock(ctypes.Structure):
    _fields_ = [("act_dtype", _c_int), ("H", _c_int), ("E", _c_int), ("K", _c_int),
                ("M", _c_int), ("L", _c_int), ("R", _c_int),
                ("router_w", _vp), ("loop_bias", _vp), ("edge_gen_w", _vp),
                ("edge_loop_bias", _vp), ("edge_value_w", _vp), ("experts", SmoeExperts),
                ("ln_w", _vp), ("ln_b", _vp), ("alpha", _c_float), ("beta", _c_float),
                ("eps", _c_float), ("edge_value_w_tiles", _vp)]


_LAYOUT_FIELDS = ["total", "logits", "top_idx", "top_w", "tok_e", "tok_ew", "e_cnt", "e_acnt",
                  "e_off", "e_rows", "e_roww", "e_tokrow", "edge_logit", "edge_idx", "edge_w",
                  "tok_d", "tok_dc", "d_cnt", "d_acnt", "d_off", "d_rows", "d_roww", "d_tokrow",
                  "proj", "msg", "act", "y", "h_tmp", "scratch", "front", "sel_idx", "sel_w", "h_tmp2"]


class SmoeWsLayout(ctypes.Structure):
    _fields_ = [(n, _sz) for n in _LAYOUT_FIELDS] + [("S", _c_int), ("ffn_dtype", _c_int)]


# every entry point of include/smoe.h: name -> (restype, argtypes)
SIGNATURES = {
    "smoe_abi_version": (_c_int, []),
    "smoe_backend_name": (ctypes.c_char_p, []),
    "smoe_backend_caps": (ctypes.c_uint32, []),
    "smoe_last_error": (ctypes.c_char_p, []),
    "smoe_block_workspace_bytes": (_sz, [ctypes.POINTER(SmoeBlock), _c_int]),
    "smoe_block_workspace_layout": (_c_int, [ctypes.POINTER(SmoeBlock), _c_int,
                                             ctypes.POINTER(SmoeWsLayout)]),
    "smoe_edge_loop_bias": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                     _vp]),
    "smoe_block_forward": (_c_int, [ctypes.POINTER(SmoeBlock), _vp, _vp, _vp, _c_int, _c_int,
                                    _c_int, _vp, _sz, _vp]),
    "smoe_block_forward_exit": (_c_int, [ctypes.POINTER(SmoeBlock), _vp, _vp, _vp, _c_int,
                                         _c_int, _c_int, _vp, ctypes.c_float, _vp, _vp, _vp, _sz,
                                         _vp]),
    "smoe_block_forward_scratch": (_c_int, [ctypes.POINTER(SmoeBlock), _vp, _vp, _vp, _c_int,
                                            _c_int, _c_int, _vp]),
    "smoe_router_workspace_bytes": (_sz, [_c_int, _c_int]),
    "smoe_router_topk": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _vp,
                                  _vp, _vp, _vp, _sz, _vp]),
    "smoe_dispatch_workspace_bytes": (_sz, [_c_int, _c_int, _c_int]),
    "smoe_dispatch_plan": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _vp, _vp, _vp, _vp, _vp,
                                    _vp, _sz, _vp]),
    "smoe_expert_delta_workspace_bytes": (_sz, [ctypes.POINTER(SmoeExperts), _c_int, _c_int]),
    "smoe_expert_delta": (_c_int, [ctypes.POINTER(SmoeExperts), _vp, _vp, _vp, _c_int, _c_int,
                                   _vp, _c_int, _vp, _sz, _vp]),
    "smoe_pack_weight_tiles": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp]),
    "smoe_pack_int4_qtiles": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "smoe_edge_topm_workspace_bytes": (_sz, [_c_int, _c_int, _c_int, _c_int]),
    "smoe_edge_topm": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _c_int, _c_int,
                                _c_int, _vp, _vp, _vp, _vp, _sz, _vp]),
    "smoe_edge_message_workspace_bytes": (_sz, [_c_int, _c_int, _c_int, _c_int, _c_int, _c_int]),
    "smoe_edge_message": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _c_int, _c_int, _c_int,
                                   _vp, _vp, _vp, _vp, _c_int, _vp, _sz, _vp]),
    "smoe_combine_epilogue": (_c_int, [_vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_float,
                                       _c_float, _vp, _vp, _c_float, _vp, _vp]),
    "smoe_select_topk": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "smoe_quantize_fp8_workspace_bytes": (_sz, []),
    "smoe_quantize_fp8_tensor": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                          _vp, _sz, _vp]),
    "smoe_linear_fp8fp8": (_c_int, [_vp, _vp, _c_int, _c_int, _vp, _vp, _vp, _c_int, _c_int, _vp,
                                    _c_int, _vp]),
    "smoe_linear": (_c_int, [_vp, _c_int, _c_int, _vp, _c_int, _vp, _vp, _c_int, _c_int, _vp,
                             _c_int, _vp]),
    "smoe_combine_rows": (_c_int, [_vp, _c_int, _vp, _vp, _c_int, _c_int, _c_int, _vp, _c_int,
                                   _vp]),
    "smoe_remap_ids": (_c_int, [_vp, ctypes.c_int64, _vp, _c_int, _vp, _vp]),
    "smoe_profile_stages": (_c_int, [ctypes.c_uint32, ctypes.POINTER(_vp), _c_int]),
    "smoe_profile_count": (_c_int, [ctypes.POINTER(ctypes.c_int32), _c_int]),
    "smoe_profile_clock": (_c_int, [_vp]),
    "smoe_events_create": (_c_int, [_c_int, ctypes.POINTER(_vp)]),
    "smoe_events_destroy": (_c_int, [_c_int, ctypes.POINTER(_vp)]),
    "smoe_events_elapsed": (_c_int, [_c_int, ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_float)]),
}

# the reference's device ABI (include/spider_cuda.h), exported by the same library
_f = ctypes.c_float
SPIDER_CUDA_SIGNATURES = {
    "spider_cuda_router_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "spider_cuda_graph_message_passing_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp,
                                                       _vp, _vp, _c_int, _c_int, _vp, _vp, _vp,
                                                       _vp]),
    "spider_cuda_expert_grouped_gemm_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                                     _vp, _vp, _vp, _vp, _vp, _vp]),
    "spider_cuda_expert_workspace_bytes": (_sz, [_c_int, _c_int, _c_int]),
    "spider_cuda_expert_grouped_gemm_v2_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int,
                                                        _c_int, _vp, _vp, _vp, _vp, _vp, _vp,
                                                        _vp]),
    "spider_cuda_loop_epilogue_f32": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _f, _f, _vp, _vp,
                                               _f, _vp, _vp]),
    "spider_cuda_early_exit_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _f, _vp, _vp]),
    "spider_cuda_moe_loop_step_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                               _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp,
                                               _vp, _vp, _f, _f, _f, _vp, _f, _vp, _vp, _vp, _vp,
                                               _vp, _vp]),
}

# this build's device-pointer forms of the reference's dynamic-edge functions
SPIDER_CUDA_SIGNATURES.update({
    "spider_cuda_edge_project_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "spider_cuda_graph_message_passing_v2_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int,
                                                          _vp, _vp, _vp, _c_int, _c_int, _vp, _vp,
                                                          _vp]),
    "spider_cuda_edge_topk_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp, _vp]),
    "spider_cuda_graph_message_passing_dynamic_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int,
                                                               _c_int, _vp, _vp, _vp, _vp, _vp]),
    "spider_cuda_edge_generator_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _vp,
                                                _vp]),
})

# the reference's host ABI (include/spider_kernels.h): host pointers
SPIDER_HOST_SIGNATURES = {
    "spider_router_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp]),
    "spider_router_f16": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp]),
    "spider_graph_message_passing_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                                  _vp, _c_int, _c_int, _vp, _vp, _vp]),
    "spider_graph_message_passing_f16": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                                  _vp, _c_int, _c_int, _vp, _vp, _vp]),
    "spider_edge_project_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "spider_graph_message_passing_v2_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _vp,
                                                     _vp, _c_int, _c_int, _vp, _vp]),
    "spider_edge_topk_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _vp]),
    "spider_graph_message_passing_dynamic_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int,
                                                          _c_int, _vp, _vp, _vp, _vp]),
    "spider_graph_dynamic_with_edge_value_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int,
                                                          _c_int, _vp, _vp, _vp, _vp, _vp, _vp]),
    "spider_edge_generator_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_int, _vp, _vp]),
    "spider_edge_generator_topk_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _vp, _c_int,
                                                _vp, _vp, _vp, _vp]),
    "spider_graph_from_generator_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp,
                                                 _c_int, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "spider_expert_grouped_gemm_f32": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp,
                                                _vp, _vp, _vp, _vp]),
    "spider_expert_grouped_gemm_f16": (_c_int, [_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _vp,
                                                _vp, _vp, _vp, _vp]),
    "spider_loop_epilogue_f32": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _f, _f, _vp, _vp, _f,
                                          _vp]),
    "spider_loop_epilogue_f16": (_c_int, [_vp, _vp, _vp, _c_int, _c_int, _f, _f, _vp, _vp, _f,
                                          _vp]),
    "spider_early_exit_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _f, _vp]),
    "spider_moe_loop_step_f32": (_c_int, [_vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp, _vp, _vp,
                                          _vp, _vp, _f, _f, _f, _vp, _f, _vp, _vp, _vp, _vp,
                                          _vp]),
    "spider_backend_name": (ctypes.c_char_p, []),
    "spider_backend_caps": (ctypes.c_uint32, []),
}

STAGES = ["router_gemm", "route_topk", "expert_plan", "edge_logits", "edge_topm", "dest_plan",
          "edge_gemm", "msg_combine", "up_gemm", "down_gemm", "epilogue",
          # stages 0-5 as one logits GEMM and its routing: bf16 steps of N <= 64
          # (one routing workgroup) and bf16 prefill at E <= 16 (the plans
          # count under expert_plan)
          "front_gemm", "front_route"]

ABI_VERSION = 10
_LIB = None


def lib():
    """The loaded library; raises when it was not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python spider-web-moe_amd/build.py` "
                "(spider_moe_amd has no CPU fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in {**SIGNATURES, **SPIDER_CUDA_SIGNATURES,
                                  **SPIDER_HOST_SIGNATURES}.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.smoe_abi_version() != ABI_VERSION:
            raise RuntimeError("libsmoe.so ABI version mismatch")
        _LIB = handle
    return _LIB


class StageTimer:
    """HIP events around every launch of the selected stages of
    smoe_block_forward (smoe_profile_stages); durations in ms per stage."""

    def __init__(self, stages=None, capacity: int = 8192, clock: bool = False):
        self.cap = capacity
        # clock: the profiled ping-pong GEMM launches also count their shader
        # clock cycles and 100 MHz wall ticks (smoe_profile_clock)
        self.clk = torch.zeros(2, dtype=torch.int64, device="cuda") if clock else None
        self.ev = (_vp * (2 * capacity))()
        check(lib().smoe_events_create(2 * capacity, self.ev), "smoe_events_create")
        ids = range(len(STAGES)) if stages is None else [STAGES.index(s) for s in stages]
        self.mask = sum(1 << i for i in ids)

    def start(self):
        check(lib().smoe_profile_stages(self.mask, self.ev, self.cap), "smoe_profile_stages")
        if self.clk is not None:
            self.clk.zero_()
            check(lib().smoe_profile_clock(self.clk.data_ptr()), "smoe_profile_clock")

    def stop(self) -> dict:
        torch.cuda.synchronize()
        stage_of = (ctypes.c_int32 * self.cap)()
        n = lib().smoe_profile_count(stage_of, self.cap)
        check(lib().smoe_profile_stages(0, None, 0), "smoe_profile_stages")
        check(lib().smoe_profile_clock(None), "smoe_profile_clock")
        ms = (ctypes.c_float * max(n, 1))()
        check(lib().smoe_events_elapsed(n, self.ev, ms), "smoe_events_elapsed")
        out: dict = {}
        for i in range(n):
            out.setdefault(STAGES[stage_of[i]], []).append(ms[i])
        return out

    def sclk_mhz(self) -> float | None:
        """The clock the profiled ping-pong GEMM tiles ran at (None when
        not counted or no such launch ran)."""
        if self.clk is None:
            return None
        c, w = (int(v) for v in self.clk.cpu())
        return 100.0 * c / w if w > 0 else None

    def close(self):
        lib().smoe_events_destroy(2 * self.cap, self.ev)


def check(rc: int, fn: str) -> None:
    """Raise RuntimeError("<fn> failed: rc") like the reference's ctypes
    wrappers (kernels/python/spider_native.py:224-225)."""
    if rc != 0:
        msg = lib().smoe_last_error().decode(errors="replace")
        raise RuntimeError(f"{fn} failed: rc={rc} ({STATUS.get(rc, '?')}): {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream_of(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(*tensors) -> torch.device:
    """All tensors on one ROCm GPU, else raise (no CPU fallback)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("spider_moe_amd runs on a ROCm GPU only; got a tensor on "
                               f"{t.device} (move the module and inputs to the GPU)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError("all tensors must be on the same GPU")
    return dev


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise RuntimeError(f"unsupported activation dtype {dt} (float32 or bfloat16)")
