"""Shared test helpers: oracle weights from a product layer, tie-aware
routing comparisons.  Quantized expert weights are decoded with the oracle's
own numpy decoders (oracle/quant.py), independently of the product code."""
from __future__ import annotations

import numpy as np
import torch

from oracle import block as B
from oracle import quant as Q

TIE_GAP = 1e-6  # routing is compared bit-exactly except where the k-th gap is below this


def oracle_weights(layer) -> B.BlockWeights:
    """float32 BlockWeights holding exactly the values the layer computes with."""
    e = layer.num_experts
    u = layer.expert_ffn_size
    f = lambda t: t.detach().float().cpu()
    w_up = torch.stack([f(m[0].weight) for m in layer.experts])
    w_down = torch.stack([f(m[2].weight) for m in layer.experts])
    b_up = b_down = None
    if layer.expert_activation == "gelu":
        b_up = torch.stack([f(m[0].bias) for m in layer.experts])
        b_down = torch.stack([f(m[2].bias) for m in layer.experts])
    fmt = layer.expert_format
    if fmt == "int4":
        qu, qd = layer._int4_w_up, layer._int4_w_down
        w_up = torch.from_numpy(Q.int4_dequantize(qu.packed.cpu().numpy(), qu.scales.float().cpu().numpy(), qu.group_size))
        w_down = torch.from_numpy(Q.int4_dequantize(qd.packed.cpu().numpy(), qd.scales.float().cpu().numpy(), qd.group_size))
        if layer._int4_b_up is not None:
            b_up, b_down = f(layer._int4_b_up), f(layer._int4_b_down)
    elif fmt == "fp8":
        cu, su, cd, sd = layer._fp8
        w_up = torch.from_numpy(Q.fp8_dequantize_per_channel(cu.cpu().view(torch.uint8).numpy(), su.cpu().numpy()))
        w_down = torch.from_numpy(Q.fp8_dequantize_per_channel(cd.cpu().view(torch.uint8).numpy(), sd.cpu().numpy()))
    w_gate = None
    if layer.expert_activation == "swiglu":
        w_gate, w_up = w_up[:, :u].contiguous(), w_up[:, u:].contiguous()
    return B.BlockWeights(
        router_w=f(layer.router.weight), loop_bias=f(layer.loop_bias),
        loop_emb=f(layer.loop_embedding.weight), edge_gen_w=f(layer.edge_generator.weight),
        edge_gen_b=f(layer.edge_generator.bias),
        edge_value_w=torch.stack([f(m.weight) for m in layer.edge_value]),
        w_up=w_up, w_down=w_down, b_up=b_up, b_down=b_down, w_gate=w_gate,
        ln_w=f(layer.norm.weight), ln_b=f(layer.norm.bias), top_k=layer.top_k,
        edges_per_expert=layer.edges_per_expert, alpha=layer.residual_scale,
        beta=layer.reinject_weight, eps=layer.norm.eps)


def routing_agrees(gpu, aux, layer, tol_gap=TIE_GAP):
    """Compare the GPU routing of the last loop with the oracle's.

    Returns (ok_tokens mask, report dict).  Tokens whose router k-th/(k+1)-th
    logit gap, or whose selected sources' m-th/(m+1)-th edge-logit gap, is
    below tol_gap are near-ties and excluded; every other token must match
    bit-exactly: top-k indices (in order), the distinct expert set, and the
    destination set.
    """
    n = aux.top_i.shape[0]
    ties = (aux.router_gap < tol_gap) | (aux.edge_gap < tol_gap)
    gi = gpu["top_idx"].long().cpu()
    same_topk = (gi == aux.top_i).all(-1)
    # destination set per token
    coef = aux.coef
    d_ref = [set(torch.nonzero(coef[t] != 0).flatten().tolist()) for t in range(n)]
    td = gpu["tok_d"].cpu()
    d_gpu = [set(x for x in td[t].tolist() if x >= 0) for t in range(n)]
    same_d = torch.tensor([a == b for a, b in zip(d_ref, d_gpu)])
    ok = same_topk & same_d
    bad = ~ok & ~ties
    return ok, {"ties": int(ties.sum()), "mismatch_non_tie": int(bad.sum()), "n": n,
                "bad_tokens": torch.nonzero(bad).flatten()[:10].tolist()}


def oracle_plan_from_topk(top_i, top_w, num_experts):
    from oracle import plan as P
    return P.dispatch_plan(top_i.numpy(), top_w.numpy(), num_experts)


def to_np(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
