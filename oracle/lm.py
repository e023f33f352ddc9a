"""Oracle: the SpiderWebLM shell around the block (TEST INFRASTRUCTURE ONLY).

Functional float32 restatement of SpiderWebLM.forward without early exit
(spider_moe/model.py:673-717) on a state dict with the reference's keys:
token embedding (model.py:357), RoPE attention prelude/coda layers
(TransformerLayer model.py:134-151, CausalSelfAttention.forward :66-74,
RoPE rope.py:8-70), the recurrent block num_loops times (:681-698), final
LayerNorm and the tied LM head (:701, :374).

Pins: golden logits written by the reference's own SpiderWebLM.forward
(tests/golden/lm_c0.npz).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import block as blk


def rope_tables(head_dim: int, max_seq: int, theta: float = 10000.0):
    """rope.py:8-27."""
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    t = torch.arange(max_seq, dtype=torch.float32)
    f = torch.outer(t, inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def _rope(x, cos, sin):
    """rope.py:30-44, 67-70 at position 0: x [B, heads, T, D]."""
    t, d = x.shape[2], x.shape[3]
    c = cos[:t].view(1, 1, t, d)
    s = sin[:t].view(1, 1, t, d)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return x * c + torch.cat([-x2, x1], dim=-1) * s


def _attention(x, sd, pre, heads, cos, sin):
    b, t, hid = x.shape
    q, k, v = (x @ sd[pre + "qkv.weight"].t()).chunk(3, dim=-1)

    def split(y):
        return y.view(b, t, heads, hid // heads).transpose(1, 2)

    q, k, v = split(q), split(k), split(v)
    if cos is not None:
        q, k = _rope(q, cos, sin), _rope(k, cos, sin)
    y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    y = y.transpose(1, 2).contiguous().view(b, t, hid)
    return y @ sd[pre + "proj.weight"].t()


def _layer(x, sd, pre, heads, cos, sin):
    hid = x.shape[-1]
    a = F.layer_norm(x, (hid,), sd[pre + "ln1.weight"], sd[pre + "ln1.bias"], 1e-5)
    x = x + _attention(a, sd, pre + "attn.", heads, cos, sin)
    f = F.layer_norm(x, (hid,), sd[pre + "ln2.weight"], sd[pre + "ln2.bias"], 1e-5)
    f = F.linear(f, sd[pre + "ffn.0.weight"], sd[pre + "ffn.0.bias"])
    f = F.gelu(f)
    f = F.linear(f, sd[pre + "ffn.2.weight"], sd[pre + "ffn.2.bias"])
    return x + f


def block_weights_from_state(sd, cfg) -> blk.BlockWeights:
    """Stack the recurrent.* parameters (model.py:172-185) into BlockWeights."""
    e = cfg["num_experts"]
    p = "recurrent."
    return blk.BlockWeights(
        router_w=sd[p + "router.weight"],
        loop_bias=sd[p + "loop_bias"],
        loop_emb=sd[p + "loop_embedding.weight"],
        edge_gen_w=sd[p + "edge_generator.weight"],
        edge_gen_b=sd[p + "edge_generator.bias"],
        edge_value_w=torch.stack([sd[f"{p}edge_value.{i}.weight"] for i in range(e)]),
        w_up=torch.stack([sd[f"{p}experts.{i}.0.weight"] for i in range(e)]),
        b_up=torch.stack([sd[f"{p}experts.{i}.0.bias"] for i in range(e)]),
        w_down=torch.stack([sd[f"{p}experts.{i}.2.weight"] for i in range(e)]),
        b_down=torch.stack([sd[f"{p}experts.{i}.2.bias"] for i in range(e)]),
        ln_w=sd[p + "norm.weight"], ln_b=sd[p + "norm.bias"],
        top_k=cfg["top_k"], edges_per_expert=cfg["edges_per_expert"],
        alpha=cfg.get("residual_scale", 0.5), beta=cfg.get("re_inject_weight", 0.1),
    )


def lm_forward(ids, sd, cfg):
    """Logits [B, T, V] of SpiderWebLM.forward(ids, early_exit=False)."""
    hid = cfg["hidden_size"]
    heads = cfg["num_heads"]
    x0 = sd["token_embedding.weight"][ids]
    cos = sin = None
    if cfg.get("use_rope", True):
        cos, sin = rope_tables(hid // heads, cfg["max_seq_len"], cfg.get("rope_theta", 10000.0))
    else:
        x0 = x0 + sd["position_embedding.weight"][: ids.shape[1]].unsqueeze(0)
    h = x0
    for i in range(cfg["num_prelude_layers"]):
        h = _layer(h, sd, f"prelude.{i}.", heads, cos, sin)
    w = block_weights_from_state(sd, cfg)
    b, t, _ = h.shape
    hf, x0f = h.reshape(b * t, hid), x0.reshape(b * t, hid)
    for r in range(cfg["num_loops"]):
        hf, _ = blk.block_forward(hf, x0f, w, r)
    h = hf.view(b, t, hid)
    for i in range(cfg["num_coda_layers"]):
        h = _layer(h, sd, f"coda.{i}.", heads, cos, sin)
    h = F.layer_norm(h, (hid,), sd["final_norm.weight"], sd["final_norm.bias"], 1e-5)
    return h @ sd["token_embedding.weight"].t()
