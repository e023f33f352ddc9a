"""spider_moe_amd — the Spider-MoE block of spider-web-moe on MI355X (gfx950).

Drop-in surface of the reference's hot path:
  SpiderMoELayer(cfg).forward(h, x0, loop_idx, return_stats=False)
  sparse_expert_delta(messages, top_indices, top_weights, w_up, b_up, w_down,
                      b_down, num_experts, top_k, expert_parallel=True)
  build_dispatch_plan / dispatch_expert_ffn
  quantize_int4 / dequantize_int4 / Int4Tensor
  forge: ForgeSelect / ForgeGEMM / ForgeEP (spider_infer/forge)
  native_compat: HipKernels / NativeLoop (the reference's spider_cuda_*
  device ABI, include/spider_cuda.h); spiderw: the .spiderw weight bundle
backed by libsmoe.so (hand-written HIP kernels, C ABI in include/smoe.h).
"""
from .config import ModelConfig, load_config
from .dispatch import DispatchPlan, ExpertAssignment, build_dispatch_plan, dispatch_expert_ffn
from .model import SpiderMoELayer, SpiderWebLM
from .quant import Int4Tensor, dequantize_int4, quantize_int4
from .sparse_experts import sparse_expert_delta
from .forge import ForgeConfig, ForgeEP, ForgeGEMM, ForgeSelect, get_forge, init_forge
from .native_compat import HipKernels, NativeLoop
from .spiderw import SpiderWBundle, SpiderWMeta, load_spiderw, write_spiderw

__all__ = ["ModelConfig", "load_config", "SpiderMoELayer", "SpiderWebLM", "sparse_expert_delta",
           "build_dispatch_plan", "dispatch_expert_ffn", "DispatchPlan", "ExpertAssignment",
           "Int4Tensor", "quantize_int4", "dequantize_int4", "ForgeConfig", "ForgeSelect",
           "ForgeGEMM", "ForgeEP", "init_forge", "get_forge", "HipKernels", "NativeLoop",
           "SpiderWBundle", "SpiderWMeta", "load_spiderw", "write_spiderw"]
