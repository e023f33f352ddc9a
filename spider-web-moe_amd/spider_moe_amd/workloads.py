"""Seeded synthetic workloads of the Spider-MoE block.

Weights: a CPU torch.Generator seeded 1000 + c draws every parameter in
named_parameters order (matrices / embeddings N(0, 0.02), biases 0,
LayerNorm weight 1, loop_bias 0); inputs: seed 2000 + c, h and x0 N(0, 1)
rounded to the activation dtype.

  c0  full SpiderWebLM forward, fp32: vocab 512, hidden 64, 4 heads,
      4 experts, top_k 2, edges 2, 2 loops, ffn 128; ids 2 x 32 in [0, 512)
  c1  prefill, bf16: H 1024, E 16, k 2, m 2, U 2816 SwiGLU, 6 loops,
      N = 8 x 2048 = 16384 tokens
  c2  decode: the c1 block with fp8-e4m3 experts (per-output-channel fp32
      scales), N = 64 x 1
  c3  skewed prefill, bf16: H 1024, E 32, k 4, m 2, U 1408 (GELU + bias),
      4 loops, N 16384; loop_bias[l, e] = log Zipf_1.2(rank(e)) over a
      seeded permutation, 4 experts forced empty with bias -1e4
  c4  int4 experts (group 128, fp16 scales): H 2048, E 64, k 2, m 4,
      U 1408 (GELU + bias), 4 loops, N = 128 decode + 2048 prefill rows
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from .config import ModelConfig
from .model import SpiderMoELayer, SpiderWebLM, init_normal_

BLOCKS = {
    "c1": dict(hidden_size=1024, num_experts=16, top_k=2, edges_per_expert=2, expert_ffn_size=2816,
               num_loops=6, expert_activation="swiglu", tokens=16384, dtype="bf16", experts="bf16"),
    "c2": dict(hidden_size=1024, num_experts=16, top_k=2, edges_per_expert=2, expert_ffn_size=2816,
               num_loops=6, expert_activation="swiglu", tokens=64, dtype="bf16", experts="fp8"),
    "c3": dict(hidden_size=1024, num_experts=32, top_k=4, edges_per_expert=2, expert_ffn_size=1408,
               num_loops=4, expert_activation="gelu", tokens=16384, dtype="bf16", experts="bf16",
               zipf=1.2, empty=4),
    "c4": dict(hidden_size=2048, num_experts=64, top_k=2, edges_per_expert=4, expert_ffn_size=1408,
               num_loops=4, expert_activation="gelu", tokens=2176, dtype="bf16", experts="int4",
               group_size=128),
}

C0 = dict(vocab_size=512, hidden_size=64, num_heads=4, num_experts=4, top_k=2, edges_per_expert=2,
          num_loops=2, expert_ffn_size=128, expert_parallel=False)

DTYPES = {"bf16": torch.bfloat16, "f32": torch.float32}


@dataclass
class BlockWorkload:
    name: str
    layer: SpiderMoELayer
    h: torch.Tensor
    x0: torch.Tensor
    spec: dict


def zipf_loop_bias(num_loops: int, num_experts: int, s: float, empty: int,
                   gen: torch.Generator) -> torch.Tensor:
    perm = torch.randperm(num_experts, generator=gen)
    rank = torch.empty(num_experts)
    rank[perm] = torch.arange(1, num_experts + 1, dtype=torch.float32)
    bias = -s * torch.log(rank)
    if empty:
        bias[perm[num_experts - empty:]] = -1e4
    return bias.view(1, -1).expand(num_loops, -1).clone()


def block_config(name: str, tokens: int | None = None, **over) -> tuple[ModelConfig, dict]:
    spec = dict(BLOCKS[name])
    spec.update(over)
    if tokens is not None:
        spec["tokens"] = tokens
    cfg = ModelConfig(vocab_size=64, num_heads=8, hidden_size=spec["hidden_size"],
                      num_experts=spec["num_experts"], top_k=spec["top_k"],
                      edges_per_expert=spec["edges_per_expert"], num_loops=spec["num_loops"],
                      expert_ffn_size=spec["expert_ffn_size"],
                      expert_activation=spec["expert_activation"], expert_parallel=False)
    return cfg.validate(), spec


def make_block(name: str, device="cuda", tokens: int | None = None, seed: int | None = None,
               std: float | str = 0.02, **over) -> BlockWorkload:
    """Build the block of workload `name` on `device` with its inputs.
    std: the weights' init scale (init_normal_; "fan_in" = 1/sqrt(fan_in))."""
    c = int(name[1:])
    cfg, spec = block_config(name, tokens, **over)
    gen = torch.Generator().manual_seed(1000 + c if seed is None else seed)
    layer = SpiderMoELayer(cfg)
    init_normal_(layer, gen, std)
    if spec.get("zipf"):
        with torch.no_grad():
            layer.loop_bias.copy_(zipf_loop_bias(cfg.num_loops, cfg.num_experts, spec["zipf"],
                                                 spec.get("empty", 0), gen))
    dt = DTYPES[spec["dtype"]]
    layer = layer.to(device=device, dtype=dt).eval()
    if spec["experts"] == "fp8":
        layer.quantize_experts_fp8()
    elif spec["experts"] == "int4":
        layer.quantize_experts(group_size=spec.get("group_size", 128), scale_dtype=torch.float16)
    ig = torch.Generator().manual_seed(2000 + c if seed is None else seed + 1000)
    n = spec["tokens"]
    h = torch.randn(n, 1, cfg.hidden_size, generator=ig).to(device=device, dtype=dt)
    x0 = torch.randn(n, 1, cfg.hidden_size, generator=ig).to(device=device, dtype=dt)
    return BlockWorkload(name=name, layer=layer, h=h, x0=x0, spec=spec)


def make_c0(device="cuda"):
    cfg = ModelConfig(**C0).validate()
    model = SpiderWebLM(cfg)
    init_normal_(model, torch.Generator().manual_seed(1000))
    ids = torch.randint(0, 512, (2, 32), generator=torch.Generator().manual_seed(2000))
    return model.to(device).eval(), ids.to(device)
