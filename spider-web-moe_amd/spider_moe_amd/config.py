"""ModelConfig: the fields of spider_moe/config.py:6-52 (same names, defaults
and validation), plus ``expert_activation`` ("gelu" = the reference's
Linear-GELU-Linear experts; "swiglu" = gated experts without biases)."""
from __future__ import annotations

from dataclasses import asdict, dataclass, fields
from pathlib import Path

import yaml


@dataclass
class ModelConfig:
    vocab_size: int = 32000
    hidden_size: int = 256
    num_heads: int = 8
    num_experts: int = 8
    top_k: int = 2
    edges_per_expert: int = 3
    num_loops: int = 6
    num_prelude_layers: int = 2
    num_coda_layers: int = 2
    expert_ffn_size: int = 512
    loop_embed_size: int = 32
    residual_scale: float = 0.5
    re_inject_weight: float = 0.1
    early_exit_threshold: float = 0.85
    dropout: float = 0.0
    embedding_init_std: float = 0.02
    max_seq_len: int = 2048
    use_rope: bool = True
    rope_theta: float = 10000.0
    expert_parallel: bool = True
    offload_experts: bool = False
    offload_max_gpu_experts: int = 4
    use_lumen: bool = False
    lumen_slots: int = 8
    lumen_slot_dim: int = 0
    lumen_j_lens: bool = True
    moe_int4: bool = False
    moe_int4_group_size: int = 64
    expert_activation: str = "gelu"

    def validate(self):
        # config.py:41-52
        if self.hidden_size % self.num_heads:
            raise ValueError("hidden_size must be divisible by num_heads")
        if not 1 <= self.top_k <= self.num_experts:
            raise ValueError("top_k must be in [1, num_experts]")
        if not 1 <= self.edges_per_expert <= self.num_experts:
            raise ValueError("edges_per_expert must be in [1, num_experts]")
        if self.num_loops < 1:
            raise ValueError("num_loops must be >= 1")
        if self.embedding_init_std <= 0:
            raise ValueError("embedding_init_std must be > 0")
        if self.expert_activation not in ("gelu", "swiglu"):
            raise ValueError("expert_activation must be 'gelu' or 'swiglu'")
        return self

    def to_dict(self):
        return asdict(self)


def load_config(path):
    """Model section of a YAML config (config.py:73-77)."""
    raw = yaml.safe_load(Path(path).read_text()) or {}
    known = {f.name for f in fields(ModelConfig)}
    model = {k: v for k, v in raw.get("model", {}).items() if k in known}
    return ModelConfig(**model).validate()
