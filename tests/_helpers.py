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


# ------------------------------------------------ value comparisons ----
# Tolerances of the intermediate values, relative to each token's largest
# reference magnitude.  The device stores the message, the FFN hidden
# activation and each expert's weighted output in bf16 (a relative error of
# 2^-9 per rounding); simulated on the CPU (tests/test_oracle_block.py::
# test_value_tolerances_are_calibrated) these give worst-token ratios below
# 0.6% for the message and 0.9% for delta, while a dropped message term, a
# dropped expert, msg = 0 or delta = 0 give ratios of 10% to 100%.
MSG_TOL = 2e-2
DELTA_TOL = 3e-2


def row_ratio(got: torch.Tensor, ref: torch.Tensor) -> torch.Tensor:
    """Per row: max |got - ref| / max |ref| (1e-30 floor)."""
    got, ref = got.float(), ref.float()
    return (got - ref).abs().amax(-1) / ref.abs().amax(-1).clamp_min(1e-30)


def gpu_delta(gpu: dict) -> torch.Tensor:
    """delta[t] = sum of y over the token's expert rows with weight > 0, in
    ascending expert order (the sum the device epilogue forms)."""
    te, tw, tr = gpu["tok_e"].long(), gpu["tok_ew"], gpu["e_tokrow"].long()
    y = gpu["y"].float()
    keep = (te >= 0) & (tw > 0)
    rows = torch.where(keep, tr, torch.zeros_like(tr))
    out = torch.zeros(te.shape[0], y.shape[1], dtype=torch.float32, device=y.device)
    for j in range(te.shape[1]):
        out += y[rows[:, j]] * keep[:, j].unsqueeze(-1).to(y.dtype)
    return out


def check_values(gpu: dict, aux, ok: torch.Tensor, sel=None, msg_tol=MSG_TOL,
                 delta_tol=DELTA_TOL) -> dict:
    """The device's message and expert delta of the last loop against the
    oracle's (aux.msg, aux.delta), on the tokens `ok` (routing-exact).  sel:
    the device token of each oracle row (a subset run), or None."""
    msg = gpu["msg"].float().cpu()
    dlt = gpu_delta(gpu).cpu()
    if sel is not None:
        msg, dlt = msg[sel], dlt[sel]
    rm = row_ratio(msg[ok], aux.msg[ok])
    rd = row_ratio(dlt[ok], aux.delta[ok])
    rep = {"msg_ratio": float(rm.max()) if rm.numel() else 0.0,
           "delta_ratio": float(rd.max()) if rd.numel() else 0.0,
           "delta_absmax": float(aux.delta[ok].abs().max()) if rd.numel() else 0.0}
    assert rep["msg_ratio"] <= msg_tol, ("message differs from the oracle", rep)
    assert rep["delta_ratio"] <= delta_tol, ("expert delta differs from the oracle", rep)
    return rep


def check_plans(gpu: dict, num_experts: int) -> None:
    """Both in-block dispatch plans, bit for bit against oracle/plan.py run on
    the device's own routing (top_idx / top_w for the experts, tok_d / tok_dc
    for the destinations), so no near-tie can make them differ.

    Expert (source) plan: every distinct selected (token, expert) pair is a
    row, experts ascending, tokens ascending inside an expert; the rows with
    merged weight > 0 are the reference's dispatch permutation, with their
    merged weights.  Destination plan: the (token, destination) pairs with a
    nonzero coefficient, destinations ascending, tokens ascending."""
    from oracle import plan as P
    e = num_experts
    top_i = gpu["top_idx"].cpu().numpy()
    top_w = gpu["top_w"].cpu().numpy()
    n, k = top_i.shape
    # all distinct pairs (the source plan the edge logits run over)
    src_rows = [np.nonzero((top_i == g).any(-1))[0] for g in range(e)]
    cnt = np.array([r.size for r in src_rows])
    assert gpu["e_cnt"].cpu().numpy().tolist() == cnt.tolist(), "source plan counts"
    off = gpu["e_off"].cpu().numpy()
    assert off.tolist() == [0] + np.cumsum(cnt).tolist(), "source plan offsets"
    rows = gpu["e_rows"].cpu().numpy()[: off[-1]]
    roww = gpu["e_roww"].cpu().numpy()[: off[-1]]
    assert rows.tolist() == (np.concatenate(src_rows).tolist() if off[-1] else []), \
        "source plan order"
    _, ocnt, operm, opw, _ = P.dispatch_plan(top_i, top_w, e)
    assert gpu["e_acnt"].cpu().numpy().tolist() == ocnt.tolist(), "dispatch counts"
    assert rows[roww > 0].tolist() == operm.tolist(), "dispatch permutation"
    assert np.array_equal(roww[roww > 0].view(np.uint32), opw.view(np.uint32)), "dispatch weights"
    # each (token, expert) entry points at its own row
    te = gpu["tok_e"].cpu().numpy()
    tr = gpu["e_tokrow"].cpu().numpy()
    for j in range(te.shape[1]):
        v = te[:, j] >= 0
        t_idx = np.nonzero(v)[0]
        r = tr[v, j]
        assert np.array_equal(rows[r], t_idx), "e_tokrow token"
        g = te[v, j]
        assert np.all((r >= off[g]) & (r < off[g + 1])), "e_tokrow group"
    # destination plan
    tok_d = gpu["tok_d"].cpu().numpy()
    tok_dc = gpu["tok_dc"].cpu().numpy()
    _, dcnt, dperm, dpw, _ = P.dispatch_plan(tok_d, tok_dc, e)
    assert gpu["d_cnt"].cpu().numpy().tolist() == dcnt.tolist(), "destination counts"
    doff = gpu["d_off"].cpu().numpy()
    assert doff.tolist() == [0] + np.cumsum(dcnt).tolist(), "destination offsets"
    drows = gpu["d_rows"].cpu().numpy()[: doff[-1]]
    assert drows.tolist() == dperm.tolist(), "destination permutation"
    droww = gpu["d_roww"].cpu().numpy()[: doff[-1]]
    assert np.array_equal(droww.view(np.uint32), dpw.view(np.uint32)), "destination weights"


def check_edges(gpu: dict, aux, ok: torch.Tensor, sel=None, w_tol=1e-5) -> int:
    """Per (token, selected source): the device's top-m destinations (in
    descending-logit order) and their softmax weights alpha against the
    oracle's edge_idx / edge_w, on the tokens `ok`; and each token's
    destination coefficients against aux.coef.  Returns the rows compared."""
    te = gpu["tok_e"].cpu()
    tr = gpu["e_tokrow"].cpu()
    eidx = gpu["edge_idx"].cpu()
    ew = gpu["edge_w"].cpu()
    tok_d, tok_dc = gpu["tok_d"].cpu(), gpu["tok_dc"].cpu()
    n = aux.top_i.shape[0]
    compared = 0
    for i in range(n):
        if not bool(ok[i]):
            continue
        t = int(sel[i]) if sel is not None else i
        for j in range(te.shape[1]):
            g = int(te[t, j])
            if g < 0:
                continue
            row = int(tr[t, j])
            assert eidx[row].tolist() == aux.edge_idx[i, g].tolist(), (t, g)
            assert torch.allclose(ew[row], aux.edge_w[i, g], rtol=0, atol=w_tol), (t, g)
            compared += 1
        d = tok_d[t]
        dv = d >= 0
        want = aux.coef[i, d[dv].long()]
        assert torch.allclose(tok_dc[t][dv], want, rtol=0, atol=w_tol), t
    return compared


def to_np(t):
    return t.detach().cpu().numpy() if isinstance(t, torch.Tensor) else np.asarray(t)
