"""Oracle: the Spider-MoE block on the CPU (TEST INFRASTRUCTURE ONLY).

A float32 restatement of SpiderMoELayer.forward (spider_moe/model.py:240-349)
and sparse_expert_delta (spider_moe/sparse_experts.py:11-68), written with
torch on the CPU because the reference's arithmetic lives in torch ops
(F.linear, softmax, topk, erf-GELU, layer_norm): using the same library keeps
op semantics (erf GELU, softmax, LayerNorm) identical by construction, while
the algorithm's structure below is restated step by step with citations.

Two formulations of the same block:

* ``faithful``  — the reference algorithm as written: dense edge projection
  over all E destinations (model.py:271-272), gather over E*m edges
  (model.py:281-288), per-expert boolean masks (sparse_experts.py:51-63).
  It is what the CPU baseline times.
* ``grouped``   — destination coefficients c[t, d] = sum of edge weights into
  d from router-selected sources, msg = sum_d c[t, d] * W_edge[d] h (the
  linearity identity of model.py:277-288), and the expert FFN over the
  dispatch plan of forge/ep/dispatch.py:56-115.  It is the GPU's algorithm
  on the CPU.

Precision contract (the reference's bf16 block raises without autocast, so
its bf16 semantics are not defined by it): weights and inputs hold values
already rounded to their storage format (bf16 / fp8 dequantized / int4
dequantized), all math is float32, and in bf16 mode the block output is
rounded to bf16.  The reference keeps messages in float32 (model.py:287-288)
and so does this oracle.

Pins (tests/test_oracle_block.py):
  * router: the reference scalar library ``spider_router_f32``
    (kernels/scalar/scalar.cpp:7-34) through oracle/_ref, and the known
    answer of kernels/tests/test_kernels.cpp:7-18;
  * edge top-m + softmax: ``spider_edge_topk_f32`` (scalar_phase1_2.cpp:11-47)
    and the known answer [2, 1] of kernels/tests/test_phase1_2.cpp:7-19;
  * edge generator logits: ``spider_edge_generator_f32``
    (scalar_phase1_3.cpp:14-42; it has no bias, so the bias is checked by
    linearity);
  * message pass: ``spider_graph_dynamic_with_edge_value_f32``
    (scalar_phase1_2.cpp:74-86) and the known answer {0, 2} of
    kernels/tests/test_phase1_2.cpp:21-32; faithful == grouped (linearity);
  * expert delta: dense all-expert einsum (the reference's own
    tests/test_sparse_experts_parity.py:41-74 construction, 1e-5), the
    duplicate-slot case (:77-98), per-token loop (tests/test_forge_04.py:30-64),
    and ``spider_expert_grouped_gemm_f32`` (scalar.cpp:55-73) with its
    tanh-GELU, no-bias, [E,H,U] conventions mapped in;
  * epilogue: ``spider_loop_epilogue_f32`` (scalar.cpp:75-92);
  * block forward: golden outputs written by the reference's own
    SpiderMoELayer.forward (tests/golden/block_*.npz).
  * SwiGLU experts are not in the reference: their parity is unpinned by the
    reference and rests on the closed form only (checked against an
    independent per-token loop).
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from . import plan as plan_mod


def round_bf16(x: torch.Tensor) -> torch.Tensor:
    """float32 values rounded to bfloat16 (RNE), returned as float32."""
    return x.to(torch.bfloat16).to(torch.float32)


@dataclass
class BlockWeights:
    """float32 parameters of one Spider-MoE block (model.py:165-185)."""

    router_w: torch.Tensor          # [E, H]        router.weight
    loop_bias: torch.Tensor         # [R, E]        loop_bias
    loop_emb: torch.Tensor          # [R, L]        loop_embedding.weight
    edge_gen_w: torch.Tensor        # [E*E, H+L]    edge_generator.weight
    edge_gen_b: torch.Tensor        # [E*E]         edge_generator.bias
    edge_value_w: torch.Tensor      # [E, H, H]     edge_value.{e}.weight
    w_up: torch.Tensor              # [E, U, H]     experts.{e}.0.weight
    w_down: torch.Tensor            # [E, H, U]     experts.{e}.2.weight
    b_up: Optional[torch.Tensor] = None    # [E, U]  experts.{e}.0.bias
    b_down: Optional[torch.Tensor] = None  # [E, H]  experts.{e}.2.bias
    w_gate: Optional[torch.Tensor] = None  # [E, U, H] SwiGLU gate (build-defined)
    ln_w: Optional[torch.Tensor] = None    # [H]
    ln_b: Optional[torch.Tensor] = None    # [H]
    top_k: int = 2
    edges_per_expert: int = 2
    alpha: float = 0.5              # residual_scale (config.py:18)
    beta: float = 0.1               # re_inject_weight (config.py:19)
    eps: float = 1e-5               # nn.LayerNorm default (model.py:184)

    @property
    def num_experts(self) -> int:
        return int(self.router_w.shape[0])

    @property
    def hidden(self) -> int:
        return int(self.router_w.shape[1])

    @property
    def act(self) -> str:
        return "swiglu" if self.w_gate is not None else "gelu"


# ------------------------------------------------------------- router ----
def router(h: torch.Tensor, w: BlockWeights, loop_idx: int):
    """model.py:255-258: logits -> fp32 softmax -> top-k on probs -> renorm.

    h: [N, H].  Returns (logits [N,E], probs [N,E], top_w [N,k], top_i [N,k]).
    """
    logits = h @ w.router_w.t() + w.loop_bias[loop_idx].view(1, -1)
    probs = logits.float().softmax(dim=-1)
    top_w, top_i = probs.topk(w.top_k, dim=-1)
    top_w = top_w / top_w.sum(dim=-1, keepdim=True).clamp_min(1e-9)
    return logits, probs, top_w, top_i


# ----------------------------------------------------- edge generator ----
def edge_logits(h: torch.Tensor, w: BlockWeights, loop_idx: int) -> torch.Tensor:
    """model.py:261-264: g = W_g [h ; loop_emb[loop]] + b_g, viewed [N, E, E]."""
    n = h.shape[0]
    e = w.num_experts
    emb = w.loop_emb[loop_idx].view(1, -1).expand(n, -1)
    g = torch.cat([h, emb], dim=-1) @ w.edge_gen_w.t() + w.edge_gen_b.view(1, -1)
    return g.view(n, e, e)


def edge_topm(g: torch.Tensor, m: int):
    """model.py:265-266: per source row, top-m on raw logits; fp32 softmax."""
    vals, idx = g.topk(m, dim=-1)
    return idx, vals.float().softmax(dim=-1)


# ------------------------------------------------------------ message ----
def message_faithful(h, w: BlockWeights, top_i, edge_idx, edge_w, chunk=2048):
    """model.py:268-288 as written: dense projection to all E destinations,
    gather at the m destinations of every source, weight by edge softmax and
    binary source activity, sum over (source, edge).  Tokens are processed in
    chunks to bound the [chunk, E, H] / [chunk, E*m, H] intermediates.
    """
    n, hid = h.shape
    e = w.num_experts
    m = edge_idx.shape[-1]
    out = torch.empty(n, hid, dtype=torch.float32)
    for s in range(0, n, chunk):
        hs = h[s:s + chunk]
        c = hs.shape[0]
        transformed = torch.einsum("nh,eoh->neo", hs, w.edge_value_w)      # :272
        active = hs.new_zeros(c, e)
        active.scatter_(-1, top_i[s:s + chunk], 1.0)                        # :277-278
        flat = edge_idx[s:s + chunk].reshape(c, e * m)                      # :281
        gathered = torch.gather(transformed, 1, flat.unsqueeze(-1).expand(c, e * m, hid))
        gathered = gathered.view(c, e, m, hid)                              # :283-284
        wt = edge_w[s:s + chunk] * active.unsqueeze(-1)                     # :287
        out[s:s + chunk] = (gathered * wt.unsqueeze(-1)).sum(dim=(1, 2))    # :288
    return out


def destination_coefficients(top_i, edge_idx, edge_w, num_experts: int) -> torch.Tensor:
    """c[t, d] = sum over distinct router-selected sources s and edges j with
    edge_idx[t, s, j] == d of edge_w[t, s, j]  (source activity is binary,
    model.py:277-278, so a source picked twice counts once)."""
    n = top_i.shape[0]
    e = num_experts
    m = edge_idx.shape[-1]
    active = torch.zeros(n, e, dtype=torch.float32)
    active.scatter_(-1, top_i, 1.0)
    wt = (edge_w * active.unsqueeze(-1)).reshape(n, e * m)
    coef = torch.zeros(n, e, dtype=torch.float32)
    coef.scatter_add_(1, edge_idx.reshape(n, e * m), wt)
    return coef


def message_grouped(h, w: BlockWeights, coef: torch.Tensor) -> torch.Tensor:
    """msg = sum_d c[:, d] * (W_edge[d] h) over tokens with c[t, d] != 0."""
    n, hid = h.shape
    out = torch.zeros(n, hid, dtype=torch.float32)
    for d in range(w.num_experts):
        rows = torch.nonzero(coef[:, d] != 0).flatten()
        if rows.numel() == 0:
            continue
        proj = h[rows] @ w.edge_value_w[d].t()
        out[rows] += coef[rows, d].unsqueeze(-1) * proj
    return out


# ------------------------------------------------------------ experts ----
def _expert_ffn(x, w: BlockWeights, e: int, act: str = "auto", hidden_bf16: bool = False):
    """hidden_bf16 rounds the FFN hidden activation to bf16 before the down
    projection, the storage the device path gives it (the reference keeps it
    in the weights' dtype, fp32 here)."""
    act = w.act if act == "auto" else act
    if act == "swiglu":
        gate = x @ w.w_gate[e].t()
        up = x @ w.w_up[e].t()
        if w.b_up is not None:
            up = up + w.b_up[e]
        hid = F.silu(gate) * up
    else:
        up = x @ w.w_up[e].t()
        if w.b_up is not None:
            up = up + w.b_up[e]
        hid = F.gelu(up) if act == "gelu" else F.gelu(up, approximate="tanh")
    if hidden_bf16:
        hid = round_bf16(hid)
    out = hid @ w.w_down[e].t()
    if w.b_down is not None:
        out = out + w.b_down[e]
    return out


def expert_delta(msg, top_i, top_w, w: BlockWeights, act: str = "auto", hidden_bf16: bool = False):
    """sparse_experts.py:45-65: for each expert, merged token weight over the
    k slots, drop weight <= 0, FFN on the active tokens, weighted add."""
    n, hid = msg.shape
    e = w.num_experts
    delta = torch.zeros(n, hid, dtype=torch.float32)
    for eid in range(e):
        tw = torch.zeros(n, dtype=torch.float32)
        for s in range(top_i.shape[1]):
            tw = tw + top_w[:, s] * (top_i[:, s] == eid).to(torch.float32)
        active = tw > 0
        if not bool(active.any()):
            continue
        out = _expert_ffn(msg[active], w, eid, act, hidden_bf16)
        delta[active] = delta[active] + out * tw[active].unsqueeze(-1)
    return delta


def expert_delta_planned(msg, top_i, top_w, w: BlockWeights, act: str = "auto"):
    """The same delta through the explicit dispatch plan
    (forge/ep/dispatch.py:145-185: pack -> FFN -> index_add)."""
    assignments, *_ = plan_mod.dispatch_plan(top_i.numpy(), top_w.numpy(), w.num_experts)
    delta = torch.zeros_like(msg, dtype=torch.float32)
    for eid, pos, wts in assignments:
        p = torch.from_numpy(pos)
        out = _expert_ffn(msg[p], w, eid, act)
        delta.index_add_(0, p, out * torch.from_numpy(wts).unsqueeze(-1))
    return delta


# ----------------------------------------------------------- epilogue ----
def epilogue(h, delta, x0, w: BlockWeights):
    """model.py:317: LayerNorm(h + alpha * delta + beta * x0), eps 1e-5."""
    hid = h.shape[-1]
    u = h + w.alpha * delta + w.beta * x0
    ln_w = w.ln_w if w.ln_w is not None else torch.ones(hid)
    ln_b = w.ln_b if w.ln_b is not None else torch.zeros(hid)
    return F.layer_norm(u, (hid,), ln_w, ln_b, w.eps)


# -------------------------------------------------------------- block ----
@dataclass
class BlockAux:
    logits: torch.Tensor
    probs: torch.Tensor
    top_w: torch.Tensor
    top_i: torch.Tensor
    edge_idx: torch.Tensor
    edge_w: torch.Tensor
    edge_gap: torch.Tensor        # per token: min over active sources of the m-th/(m+1)-th logit gap
    router_gap: torch.Tensor      # per token: k-th/(k+1)-th logit gap
    msg: torch.Tensor
    delta: torch.Tensor
    coef: torch.Tensor
    extra: dict = field(default_factory=dict)


def _kth_gap(x: torch.Tensor, k: int) -> torch.Tensor:
    """Gap between the k-th and (k+1)-th largest value along the last dim
    (+inf when there is no (k+1)-th)."""
    if x.shape[-1] <= k:
        return torch.full(x.shape[:-1], float("inf"))
    v = x.topk(k + 1, dim=-1).values
    return (v[..., k - 1] - v[..., k]).abs()


def block_forward(h, x0, w: BlockWeights, loop_idx: int, *, mode: str = "faithful",
                  out_bf16: bool = False, act: str = "auto", chunk: int = 2048):
    """One loop of the block.  h, x0: [N, H] float32.  Returns (h', aux)."""
    h = h.float()
    x0 = x0.float()
    logits, probs, top_w, top_i = router(h, w, loop_idx)
    n = h.shape[0]
    e = w.num_experts
    m = w.edges_per_expert
    # edge logits: computed in token chunks (N x E*E can be large)
    edge_idx = torch.empty(n, e, m, dtype=torch.long)
    edge_w = torch.empty(n, e, m, dtype=torch.float32)
    edge_gap = torch.empty(n, dtype=torch.float32)
    for s in range(0, n, chunk):
        g = edge_logits(h[s:s + chunk], w, loop_idx)
        ei, ew = edge_topm(g, m)
        edge_idx[s:s + chunk] = ei
        edge_w[s:s + chunk] = ew
        gaps = _kth_gap(g, m)                                   # [c, E]
        sel = torch.zeros_like(gaps, dtype=torch.bool)
        sel.scatter_(-1, top_i[s:s + chunk], True)
        edge_gap[s:s + chunk] = torch.where(sel, gaps, torch.full_like(gaps, float("inf"))).amin(-1)
    coef = destination_coefficients(top_i, edge_idx, edge_w, e)
    if mode == "faithful":
        msg = message_faithful(h, w, top_i, edge_idx, edge_w, chunk=chunk)
        delta = expert_delta(msg, top_i, top_w, w, act)
    elif mode == "grouped":
        msg = message_grouped(h, w, coef)
        delta = expert_delta_planned(msg, top_i, top_w, w, act)
    else:
        raise ValueError(mode)
    out = epilogue(h, delta, x0, w)
    if out_bf16:
        out = round_bf16(out)
    aux = BlockAux(logits=logits, probs=probs, top_w=top_w, top_i=top_i,
                   edge_idx=edge_idx, edge_w=edge_w, edge_gap=edge_gap,
                   router_gap=_kth_gap(logits, w.top_k), msg=msg, delta=delta, coef=coef)
    return out, aux


def block_stats(aux: BlockAux, num_experts: int, out, exit_w, exit_b, *, logit_bf16: bool = False):
    """The return_stats branch of model.py:327-345 over one loop's routing
    (aux of block_forward, every source's top-m edges) and its output h'
    [N, H]: expert / edge load (bincount over top-k / every edge,
    normalised by max(sum, 1)), edge importance (scatter-add of the edge
    softmax weights, normalised by max(sum, 1e-9)), aux_loss =
    E * sum(load * mean_t probs), edge_loss = E * sum(edge_load *
    importance), confidence = sigmoid(exit_head(h')) [N]."""
    e = int(num_experts)
    load = torch.bincount(aux.top_i.reshape(-1), minlength=e).float()
    load = load / load.sum().clamp_min(1.0)
    edge_load = torch.bincount(aux.edge_idx.reshape(-1), minlength=e).float()
    edge_load = edge_load / edge_load.sum().clamp_min(1.0)
    imp = torch.zeros(e, dtype=torch.float32).scatter_add(0, aux.edge_idx.reshape(-1),
                                                            aux.edge_w.reshape(-1).float())
    imp = imp / imp.sum().clamp_min(1e-9)
    probs_mean = aux.probs.reshape(-1, e).mean(dim=0)
    return {
        "expert_load": load,
        "edge_load": edge_load,
        "aux_loss": e * torch.sum(load * probs_mean),
        "edge_loss": e * torch.sum(edge_load * imp),
        "confidence": torch.sigmoid(exit_logit(out, exit_w, exit_b, bf16=logit_bf16)),
    }


def block_loops(h, x0, w: BlockWeights, num_loops: int, **kw):
    """model.py:445-448: run the shared block num_loops times."""
    for r in range(num_loops):
        h, _ = block_forward(h, x0, w, r, **kw)
    return h


def exit_logit(h, exit_w, exit_b, bf16: bool = False):
    """exit_head(h) (model.py:185,467): h . w + b in float32; the confidence
    is its sigmoid.  bf16: the exit head of a bf16 model is a bf16 Linear,
    whose output is rounded to bf16 before `.float()` and the sigmoid."""
    z = h.float() @ exit_w.float().reshape(-1) + float(exit_b)
    return round_bf16(z) if bf16 else z


def block_loops_exit(h, x0, w: BlockWeights, num_loops: int, exit_w, exit_b, threshold: float,
                     *, loop_begin: int = 0, logit_bf16: bool = False, **kw):
    """Early-exit decode: SpiderWebLM._run_recurrent_decode(early_exit=True)
    (model.py:450-473) over the ActiveSet compaction of active_set.py:14-64.
    Each loop gathers the rows still in orbit (compact_active: index_select),
    runs the block on them, writes them back (scatter_active: index_copy_)
    and drops the rows whose sigmoid(exit_head(h')) > threshold
    (ActiveSet.drop); the loop stops when no row is left (model.py:461-462).

    Returns (h [N, H], loops [N] = loops each row ran, margin [N] = the
    smallest |exit logit - logit(threshold)| over the loops a row ran: rows
    with a tiny margin are near-ties of the exit decision)."""
    h = h.float().clone()
    x0 = x0.float()
    n = h.shape[0]
    idx = torch.arange(n)
    loops = torch.zeros(n, dtype=torch.long)
    margin = torch.full((n,), float("inf"))
    if 0.0 < threshold < 1.0:
        z_thr = float(np.log(threshold / (1.0 - threshold)))
    else:
        z_thr = float("inf") if threshold >= 1.0 else float("-inf")
    for r in range(loop_begin, loop_begin + num_loops):
        if idx.numel() == 0:
            break
        h_new, _ = block_forward(h.index_select(0, idx), x0.index_select(0, idx), w, r, **kw)
        h.index_copy_(0, idx, h_new)
        z = exit_logit(h_new, exit_w, exit_b, bf16=logit_bf16)
        loops[idx] += 1
        margin[idx] = torch.minimum(margin[idx], (z - z_thr).abs())
        idx = idx[~(torch.sigmoid(z) > threshold)]
    return h, loops, margin
