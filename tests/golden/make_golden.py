"""Write the golden fixtures of tests/golden/ from the reference's own code.

Run in the development container only (the reference is absent elsewhere):

    python tests/golden/make_golden.py [/path/to/reference]

It imports the reference's ``spider_moe`` package (model.py, quant.py,
sparse_experts.py) to record input/output vectors for what the oracle's other
checks leave open: the composition of SpiderMoELayer.forward
(spider_moe/model.py:240-349), SpiderWebLM.forward (model.py:673-717),
sparse_expert_delta with duplicate / zero / negative slot weights
(sparse_experts.py:11-68) and the quantize_int4 bytes (quant.py:89-117).
Only data (inputs, parameters, outputs) is written: .npz files, float32 /
int64 / uint8 arrays.  Single-threaded torch for reproducibility.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _np(t):
    return t.detach().cpu().numpy()


def _init_normal(model, seed, std=0.02):
    """Re-draw every parameter: matrices/embeddings N(0, std) in state-dict
    order, biases 0, LayerNorm weight 1, loop_bias 0."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("loop_bias"):
                p.zero_()
            elif ".norm." in name or "ln1" in name or "ln2" in name or "final_norm" in name:
                p.fill_(1.0 if name.endswith("weight") else 0.0)
            elif name.endswith("bias"):
                p.zero_()
            else:
                p.copy_(torch.randn(p.shape, generator=g) * std)


def block_fixture(ref, name, cfg_kw, n_b, n_t, seed, std, loop_bias_std=0.0, bias_std=0.0):
    from spider_moe.config import ModelConfig
    from spider_moe.model import SpiderMoELayer

    cfg = ModelConfig(**cfg_kw).validate()
    layer = SpiderMoELayer(cfg).eval()
    _init_normal(layer, seed, std)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        if loop_bias_std:
            layer.loop_bias.copy_(torch.randn(layer.loop_bias.shape, generator=g) * loop_bias_std)
        if bias_std:
            layer.edge_generator.bias.copy_(
                torch.randn(layer.edge_generator.bias.shape, generator=g) * bias_std)
            for ex in layer.experts:
                ex[0].bias.copy_(torch.randn(ex[0].bias.shape, generator=g) * bias_std)
                ex[2].bias.copy_(torch.randn(ex[2].bias.shape, generator=g) * bias_std)
            layer.norm.weight.copy_(1.0 + torch.randn(layer.norm.weight.shape, generator=g) * 0.1)
            layer.norm.bias.copy_(torch.randn(layer.norm.bias.shape, generator=g) * 0.1)
    h = torch.randn(n_b, n_t, cfg.hidden_size, generator=g)
    x0 = torch.randn(n_b, n_t, cfg.hidden_size, generator=g)
    out = {f"param/{k}": _np(v) for k, v in layer.state_dict().items()}
    out["h"] = _np(h)
    out["x0"] = _np(x0)
    out["cfg/hidden_size"] = np.int64(cfg.hidden_size)
    out["cfg/num_experts"] = np.int64(cfg.num_experts)
    out["cfg/top_k"] = np.int64(cfg.top_k)
    out["cfg/edges_per_expert"] = np.int64(cfg.edges_per_expert)
    out["cfg/num_loops"] = np.int64(cfg.num_loops)
    out["cfg/expert_ffn_size"] = np.int64(cfg.expert_ffn_size)
    out["cfg/loop_embed_size"] = np.int64(cfg.loop_embed_size)
    with torch.no_grad():
        cur = h
        for r in range(cfg.num_loops):
            # teacher-forced: each loop's input is the previous reference output
            y, stats = layer(cur, x0, r, return_stats=True)
            out[f"loop{r}/in"] = _np(cur)
            out[f"loop{r}/out"] = _np(y)
            out[f"loop{r}/router_probs"] = _np(stats["router_probs"])
            out[f"loop{r}/expert_load"] = _np(stats["expert_load"])
            out[f"loop{r}/edge_load"] = _np(stats["edge_load"])
            out[f"loop{r}/aux_loss"] = _np(stats["aux_loss"])
            out[f"loop{r}/edge_loss"] = _np(stats["edge_loss"])
            cur = y
        # int4 experts (quantize_experts, model.py:218-231) on the loop-0 input
        layer.quantize_experts(group_size=cfg_kw.get("moe_int4_group_size", 16))
        y4 = layer(h, x0, 0)
        out["int4/group_size"] = np.int64(layer._int4_w_up.group_size)
        out["int4/w_up_packed"] = _np(layer._int4_w_up.packed)
        out["int4/w_up_scales"] = _np(layer._int4_w_up.scales)
        out["int4/w_down_packed"] = _np(layer._int4_w_down.packed)
        out["int4/w_down_scales"] = _np(layer._int4_w_down.scales)
        out["int4/loop0_out"] = _np(y4)
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print("wrote", name, {k: v.shape for k, v in out.items() if k.startswith("loop0")})


def sparse_delta_fixture():
    from spider_moe.sparse_experts import sparse_expert_delta

    g = torch.Generator().manual_seed(31)
    b, t, h, e, k, u = 2, 6, 16, 5, 3, 24
    msg = torch.randn(b, t, h, generator=g)
    idx = torch.randint(0, e, (b, t, k), generator=g)
    idx[0, 0] = torch.tensor([2, 2, 2])          # triple duplicate
    idx[0, 1] = torch.tensor([1, 3, 1])          # duplicate
    w = torch.rand(b, t, k, generator=g)
    w[0, 2, 1] = 0.0                             # zero weight slot
    w[1, 3] = torch.tensor([0.5, -0.5, 0.25])    # negative weight slot
    idx[1, 3] = torch.tensor([4, 4, 0])          # merged weight 0 -> dropped
    w_up = torch.randn(e, u, h, generator=g) * 0.2
    b_up = torch.randn(e, u, generator=g) * 0.1
    w_down = torch.randn(e, h, u, generator=g) * 0.2
    b_down = torch.randn(e, h, generator=g) * 0.1
    d = sparse_expert_delta(msg, idx, w, w_up, b_up, w_down, b_down,
                            num_experts=e, top_k=k, expert_parallel=False)
    np.savez_compressed(os.path.join(HERE, "sparse_delta.npz"), msg=_np(msg), idx=_np(idx),
                        w=_np(w), w_up=_np(w_up), b_up=_np(b_up), w_down=_np(w_down),
                        b_down=_np(b_down), delta=_np(d))
    print("wrote sparse_delta")


def int4_fixture():
    from spider_moe.quant import quantize_int4

    g = torch.Generator().manual_seed(41)
    w = torch.randn(4, 256, generator=g)
    w[0, :8] = torch.tensor([0.0, 1.0, -1.0, 0.5, -0.5, 0.25, 3.5, -3.5])
    out = {"w": _np(w)}
    for gs in (32, 64, 128, 48):  # 48 does not divide 256 -> whole-row group
        q = quantize_int4(w, group_size=gs)
        out[f"g{gs}/packed"] = _np(q.packed)
        out[f"g{gs}/scales"] = _np(q.scales)
        out[f"g{gs}/group"] = np.int64(q.group_size)
        out[f"g{gs}/deq"] = _np(q.dequantize(dtype=torch.float32))
    np.savez_compressed(os.path.join(HERE, "quant_int4.npz"), **out)
    print("wrote quant_int4")


def lm_fixture():
    from spider_moe.config import ModelConfig
    from spider_moe.model import SpiderWebLM

    kw = dict(vocab_size=512, hidden_size=64, num_heads=4, num_experts=4, top_k=2,
              edges_per_expert=2, num_loops=2, expert_ffn_size=128, expert_parallel=False)
    cfg = ModelConfig(**kw).validate()
    model = SpiderWebLM(cfg).eval()
    _init_normal(model, 1000)
    g = torch.Generator().manual_seed(2000)
    ids = torch.randint(0, 512, (2, 32), generator=g)
    with torch.no_grad():
        logits = model(ids, early_exit=False)["logits"]
    # lm_head is tied to token_embedding; the absolute position table is
    # unused with RoPE (model.py:392-404)
    out = {f"param/{k}": _np(v) for k, v in model.state_dict().items()
           if not k.startswith("lm_head") and not k.startswith("position_embedding")}
    out["ids"] = _np(ids)
    out["logits"] = _np(logits)
    for k, v in kw.items():
        out[f"cfg/{k}"] = np.int64(v)
    np.savez_compressed(os.path.join(HERE, "lm_c0.npz"), **out)
    print("wrote lm_c0", logits.shape)


def main():
    ref = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, ref)
    torch.set_num_threads(1)
    torch.use_deterministic_algorithms(True)
    block_fixture(ref, "block_small",
                  dict(vocab_size=64, hidden_size=32, num_heads=4, num_experts=4, top_k=2,
                       edges_per_expert=2, num_loops=2, expert_ffn_size=64, loop_embed_size=8,
                       expert_parallel=False, moe_int4_group_size=16),
                  2, 8, seed=11, std=0.2)
    block_fixture(ref, "block_mid",
                  dict(vocab_size=64, hidden_size=64, num_heads=4, num_experts=8, top_k=3,
                       edges_per_expert=3, num_loops=3, expert_ffn_size=96, loop_embed_size=16,
                       expert_parallel=False, moe_int4_group_size=32),
                  3, 16, seed=12, std=0.1, loop_bias_std=0.5, bias_std=0.1)
    sparse_delta_fixture()
    int4_fixture()
    lm_fixture()


if __name__ == "__main__":
    main()
