"""Pins for oracle/block.py and oracle/lm.py: the reference's scalar C++
library (compiled from its sources into oracle/_ref), the reference's own
known-answer tests, golden outputs of the reference's SpiderMoELayer /
SpiderWebLM / sparse_expert_delta, and closed-form identities."""
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import GOLDEN
from oracle import block as B
from oracle import lm as LM
from oracle import ref as R

needs_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built")


def load_block(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    sd = {k[len("param/"):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param/")}
    cfg = {k[len("cfg/"):]: int(z[k]) for k in z.files if k.startswith("cfg/")}
    e = cfg["num_experts"]
    w = B.BlockWeights(
        router_w=sd["router.weight"], loop_bias=sd["loop_bias"],
        loop_emb=sd["loop_embedding.weight"], edge_gen_w=sd["edge_generator.weight"],
        edge_gen_b=sd["edge_generator.bias"],
        edge_value_w=torch.stack([sd[f"edge_value.{i}.weight"] for i in range(e)]),
        w_up=torch.stack([sd[f"experts.{i}.0.weight"] for i in range(e)]),
        b_up=torch.stack([sd[f"experts.{i}.0.bias"] for i in range(e)]),
        w_down=torch.stack([sd[f"experts.{i}.2.weight"] for i in range(e)]),
        b_down=torch.stack([sd[f"experts.{i}.2.bias"] for i in range(e)]),
        ln_w=sd["norm.weight"], ln_b=sd["norm.bias"],
        top_k=cfg["top_k"], edges_per_expert=cfg["edges_per_expert"])
    return z, w, cfg


# --------------------------------------------------- reference goldens ----
@pytest.mark.parametrize("name", ["block_small", "block_mid"])
@pytest.mark.parametrize("mode", ["faithful", "grouped"])
def test_block_matches_reference_layer(name, mode):
    z, w, cfg = load_block(name)
    hid = cfg["hidden_size"]
    x0 = torch.from_numpy(z["x0"]).reshape(-1, hid)
    for r in range(cfg["num_loops"]):
        h = torch.from_numpy(z[f"loop{r}/in"]).reshape(-1, hid)
        out, aux = B.block_forward(h, x0, w, r, mode=mode)
        ref = torch.from_numpy(z[f"loop{r}/out"]).reshape(-1, hid)
        torch.testing.assert_close(out, ref, rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(aux.probs, torch.from_numpy(z[f"loop{r}/router_probs"]).reshape(-1, cfg["num_experts"]), rtol=1e-6, atol=1e-7)
        load = torch.bincount(aux.top_i.reshape(-1), minlength=cfg["num_experts"]).float()
        load = load / load.sum()
        assert torch.equal(load, torch.from_numpy(z[f"loop{r}/expert_load"]))
        eload = torch.bincount(aux.edge_idx.reshape(-1), minlength=cfg["num_experts"]).float()
        assert torch.equal(eload / eload.sum(), torch.from_numpy(z[f"loop{r}/edge_load"]))


@pytest.mark.parametrize("name", ["block_small", "block_mid"])
def test_block_stats_match_reference_layer(name):
    """block_stats against the return_stats outputs the reference's layer
    wrote (model.py:327-345): loads bit for bit, aux_loss / edge_loss to
    float32 rounding; planted mistakes (load normalised per token instead
    of per slot, probs summed instead of averaged, edge importance without
    its softmax weights) miss the goldens."""
    z, w, cfg = load_block(name)
    hid, e = cfg["hidden_size"], cfg["num_experts"]
    x0 = torch.from_numpy(z["x0"]).reshape(-1, hid)
    ew = torch.from_numpy(z["param/exit_head.weight"]).reshape(-1)
    eb = float(z["param/exit_head.bias"].reshape(-1)[0])
    for r in range(cfg["num_loops"]):
        h = torch.from_numpy(z[f"loop{r}/in"]).reshape(-1, hid)
        out, aux = B.block_forward(h, x0, w, r)
        st = B.block_stats(aux, e, out, ew, eb)
        assert torch.equal(st["expert_load"], torch.from_numpy(z[f"loop{r}/expert_load"]))
        assert torch.equal(st["edge_load"], torch.from_numpy(z[f"loop{r}/edge_load"]))
        for key in ("aux_loss", "edge_loss"):
            ref = torch.from_numpy(np.asarray(z[f"loop{r}/{key}"], dtype=np.float32)).reshape(())
            torch.testing.assert_close(st[key].reshape(()), ref, rtol=1e-6, atol=1e-7)
        n = h.shape[0]
        ref_aux = float(z[f"loop{r}/aux_loss"])
        per_token = st["expert_load"] * w.top_k  # bincount / N
        assert abs(float(e * torch.sum(per_token * aux.probs.mean(0))) - ref_aux) > 1e-3
        assert abs(float(e * torch.sum(st["expert_load"] * aux.probs.sum(0))) - ref_aux) > 1e-3
        flat = torch.bincount(aux.edge_idx.reshape(-1), minlength=e).float()
        ref_edge = float(z[f"loop{r}/edge_loss"])
        assert abs(float(e * torch.sum(st["edge_load"] * flat / flat.sum())) - ref_edge) > 1e-5
        assert st["confidence"].shape == (n,)


def test_block_stats_confidence_known_answer():
    """confidence = sigmoid(exit_head(h')) on the block's output: with the
    exit head reading feature 0, h'[:, 0] = 0, ln 3, -ln 3 give 1/2, 3/4,
    1/4; the bias shifts the logit (model.py:342, exit_head model.py:185)."""
    out = torch.zeros(3, 4)
    out[:, 0] = torch.tensor([0.0, float(np.log(3.0)), -float(np.log(3.0))])
    ew = torch.tensor([1.0, 0.0, 0.0, 0.0])
    aux = B.BlockAux(logits=torch.zeros(3, 2), probs=torch.full((3, 2), 0.5),
                     top_w=torch.ones(3, 1), top_i=torch.zeros(3, 1, dtype=torch.long),
                     edge_idx=torch.zeros(3, 2, 1, dtype=torch.long), edge_w=torch.ones(3, 2, 1),
                     edge_gap=torch.zeros(3), router_gap=torch.zeros(3), msg=out, delta=out,
                     coef=torch.zeros(3, 2))
    conf = B.block_stats(aux, 2, out, ew, 0.0)["confidence"]
    torch.testing.assert_close(conf, torch.tensor([0.5, 0.75, 0.25]), rtol=0, atol=1e-7)
    shifted = B.block_stats(aux, 2, out, ew, float(np.log(3.0)))["confidence"]
    torch.testing.assert_close(shifted[0], torch.tensor(0.75), rtol=0, atol=1e-7)
    # aux_loss of uniform probs and all load on expert 0: E * 1 * 1/2 = 1
    st = B.block_stats(aux, 2, out, ew, 0.0)
    assert float(st["aux_loss"]) == 1.0 and float(st["edge_loss"]) == 2.0


@pytest.mark.parametrize("name", ["block_small", "block_mid"])
def test_block_int4_matches_reference_layer(name):
    from oracle import quant as Q
    z, w, cfg = load_block(name)
    hid = cfg["hidden_size"]
    g = int(z["int4/group_size"])
    pu, su, g1 = Q.int4_quantize(w.w_up.numpy(), g)
    pd, sd_, g2 = Q.int4_quantize(w.w_down.numpy(), g)
    assert np.array_equal(pu, z["int4/w_up_packed"]) and np.array_equal(pd, z["int4/w_down_packed"])
    assert np.array_equal(su, z["int4/w_up_scales"]) and np.array_equal(sd_, z["int4/w_down_scales"])
    w.w_up = torch.from_numpy(Q.int4_dequantize(pu, su, g1))
    w.w_down = torch.from_numpy(Q.int4_dequantize(pd, sd_, g2))
    h = torch.from_numpy(z["h"]).reshape(-1, hid)
    x0 = torch.from_numpy(z["x0"]).reshape(-1, hid)
    out, _ = B.block_forward(h, x0, w, 0)
    torch.testing.assert_close(out, torch.from_numpy(z["int4/loop0_out"]).reshape(-1, hid), rtol=1e-5, atol=1e-5)


def test_sparse_delta_matches_reference_with_duplicates_and_nonpositive():
    z = np.load(os.path.join(GOLDEN, "sparse_delta.npz"))
    t = {k: torch.from_numpy(z[k]) for k in z.files}
    e = t["w_up"].shape[0]
    hid = t["msg"].shape[-1]
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(1, e),
                       loop_emb=torch.zeros(1, 1), edge_gen_w=torch.zeros(e * e, hid + 1),
                       edge_gen_b=torch.zeros(e * e), edge_value_w=torch.zeros(e, hid, hid),
                       w_up=t["w_up"], b_up=t["b_up"], w_down=t["w_down"], b_down=t["b_down"])
    k = t["idx"].shape[-1]
    msg = t["msg"].reshape(-1, hid)
    idx = t["idx"].reshape(-1, k)
    wt = t["w"].reshape(-1, k)
    ref = t["delta"].reshape(-1, hid)
    torch.testing.assert_close(B.expert_delta(msg, idx, wt, w), ref, rtol=1e-6, atol=1e-6)
    torch.testing.assert_close(B.expert_delta_planned(msg, idx, wt, w), ref, rtol=1e-5, atol=1e-5)


def test_lm_c0_matches_reference_forward():
    z = np.load(os.path.join(GOLDEN, "lm_c0.npz"))
    sd = {k[len("param/"):]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param/")}
    cfg = {k[len("cfg/"):]: int(z[k]) for k in z.files if k.startswith("cfg/")}
    cfg.update(num_prelude_layers=2, num_coda_layers=2, max_seq_len=2048, use_rope=True)
    logits = LM.lm_forward(torch.from_numpy(z["ids"]), sd, cfg)
    torch.testing.assert_close(logits, torch.from_numpy(z["logits"]), rtol=1e-4, atol=1e-5)


# ------------------------------------------ reference scalar C++ library ----
@needs_ref
def test_router_matches_scalar_library():
    rng = np.random.default_rng(5)
    n, hid, e, k, loops = 64, 32, 8, 3, 3
    h = torch.from_numpy(rng.standard_normal((n, hid)).astype(np.float32))
    w = B.BlockWeights(router_w=torch.from_numpy(rng.standard_normal((e, hid)).astype(np.float32) * 0.3),
                       loop_bias=torch.from_numpy(rng.standard_normal((loops, e)).astype(np.float32)),
                       loop_emb=torch.zeros(loops, 1), edge_gen_w=torch.zeros(e * e, hid + 1),
                       edge_gen_b=torch.zeros(e * e), edge_value_w=torch.zeros(e, hid, hid),
                       w_up=torch.zeros(e, 4, hid), w_down=torch.zeros(e, hid, 4), top_k=k)
    for r in range(loops):
        logits, probs, tw, ti = B.router(h, w, r)
        raw = (h @ w.router_w.t()).numpy()
        rc, rw, ri = R.router_f32(raw, w.loop_bias.numpy(), k, r)
        assert rc == 0
        assert np.array_equal(ti.numpy(), ri)
        np.testing.assert_allclose(tw.numpy(), rw, rtol=1e-5, atol=1e-7)


@needs_ref
def test_router_known_answer_and_invalid_args():
    # kernels/tests/test_kernels.cpp:7-18, :57-59
    logits = np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float32)
    rc, rw, ri = R.router_f32(logits, np.zeros((1, 4), np.float32), 2, 0)
    assert rc == 0 and ri.tolist() == [[3, 2], [0, 1]]
    assert np.allclose(rw.sum(-1), 1.0)
    w = B.BlockWeights(router_w=torch.eye(4), loop_bias=torch.zeros(1, 4), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(16, 5), edge_gen_b=torch.zeros(16),
                       edge_value_w=torch.zeros(4, 4, 4), w_up=torch.zeros(4, 4, 4),
                       w_down=torch.zeros(4, 4, 4), top_k=2)
    _, _, tw, ti = B.router(torch.from_numpy(logits), w, 0)
    assert ti.tolist() == [[3, 2], [0, 1]]
    np.testing.assert_allclose(tw.numpy(), rw, rtol=1e-6)
    assert R.lib().spider_router_f32(None, None, 0, 0, 0, 0, None, None) != 0


@needs_ref
def test_edge_topm_matches_scalar_library():
    rng = np.random.default_rng(6)
    g = torch.from_numpy(rng.standard_normal((40, 6, 6)).astype(np.float32))
    for m in (1, 2, 3):
        idx, ew = B.edge_topm(g, m)
        rc, ri, rw = R.edge_topk_f32(g.numpy(), m)
        assert rc == 0
        assert np.array_equal(idx.numpy(), ri)
        np.testing.assert_allclose(ew.numpy(), rw, rtol=1e-6, atol=1e-7)
    # known answer kernels/tests/test_phase1_2.cpp:7-19
    kg = torch.tensor([[[0., 1., 2.], [3., 0., 1.], [0., 0., 1.]]])
    idx, ew = B.edge_topm(kg, 2)
    assert idx[0, 0].tolist() == [2, 1] and abs(float(ew[0, 0].sum()) - 1) < 1e-6


@needs_ref
def test_edge_generator_matches_scalar_library_plus_bias_by_linearity():
    rng = np.random.default_rng(7)
    n, hid, e, lemb = 16, 24, 5, 6
    h = torch.from_numpy(rng.standard_normal((n, hid)).astype(np.float32))
    wg = torch.from_numpy(rng.standard_normal((e * e, hid + lemb)).astype(np.float32) * 0.2)
    bg = torch.from_numpy(rng.standard_normal(e * e).astype(np.float32))
    emb = torch.from_numpy(rng.standard_normal((2, lemb)).astype(np.float32))
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(2, e), loop_emb=emb,
                       edge_gen_w=wg, edge_gen_b=bg, edge_value_w=torch.zeros(e, hid, hid),
                       w_up=torch.zeros(e, 4, hid), w_down=torch.zeros(e, hid, 4))
    for r in range(2):
        ours = B.edge_logits(h, w, r)
        rc, theirs = R.edge_generator_f32(h.numpy(), emb[r].numpy(), wg.numpy())
        assert rc == 0
        np.testing.assert_allclose((ours - bg.view(1, e, e)).numpy(), theirs, rtol=1e-5, atol=1e-5)


@needs_ref
def test_message_matches_scalar_library_and_linearity():
    rng = np.random.default_rng(8)
    n, hid, e, k, m = 24, 16, 6, 2, 3
    h = torch.from_numpy(rng.standard_normal((n, hid)).astype(np.float32))
    we = torch.from_numpy(rng.standard_normal((e, hid, hid)).astype(np.float32) * 0.3)
    g = torch.from_numpy(rng.standard_normal((n, e, e)).astype(np.float32))
    ei, ew = B.edge_topm(g, m)
    ti = torch.stack([torch.randperm(e, generator=torch.Generator().manual_seed(i))[:k] for i in range(n)])
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(1, e), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(e * e, hid + 1), edge_gen_b=torch.zeros(e * e),
                       edge_value_w=we, w_up=torch.zeros(e, 4, hid), w_down=torch.zeros(e, hid, 4))
    faithful = B.message_faithful(h, w, ti, ei, ew)
    rc, theirs = R.graph_dynamic_with_edge_value_f32(h.numpy(), we.numpy(), ei.numpy(), ew.numpy(), ti.numpy())
    assert rc == 0
    np.testing.assert_allclose(faithful.numpy(), theirs, rtol=1e-5, atol=1e-5)
    coef = B.destination_coefficients(ti, ei, ew, e)
    torch.testing.assert_close(B.message_grouped(h, w, coef), faithful, rtol=1e-5, atol=1e-5)
    # each active source's edge weights sum to 1 -> coefficients sum to k
    torch.testing.assert_close(coef.sum(-1), torch.full((n,), float(k)), rtol=1e-6, atol=1e-6)
    # known answer kernels/tests/test_phase1_2.cpp:21-32: projections
    # P[0] = [1, 0], P[1] = [0, 4]; source 0's only edge goes to 1 with
    # weight 0.5 -> message [0, 2].  P = W_e h with h = [1, 0].
    h1 = torch.tensor([[1.0, 0.0]])
    we1 = torch.stack([torch.eye(2), torch.tensor([[0.0, 0.0], [4.0, 0.0]])])
    w1 = B.BlockWeights(router_w=torch.zeros(2, 2), loop_bias=torch.zeros(1, 2), loop_emb=torch.zeros(1, 1),
                        edge_gen_w=torch.zeros(4, 3), edge_gen_b=torch.zeros(4), edge_value_w=we1,
                        w_up=torch.zeros(2, 4, 2), w_down=torch.zeros(2, 2, 4), top_k=1, edges_per_expert=1)
    ei1 = torch.tensor([[[1], [0]]])
    ew1 = torch.tensor([[[0.5], [1.0]]])
    msg1 = B.message_faithful(h1, w1, torch.tensor([[0]]), ei1, ew1)
    assert msg1.tolist() == [[0.0, 2.0]]
    rc, msg1r = R.graph_dynamic_with_edge_value_f32(h1.numpy(), we1.numpy(), ei1.numpy(), ew1.numpy(), np.array([[0]]))
    assert rc == 0 and msg1r.tolist() == [[0.0, 2.0]]


@needs_ref
def test_expert_delta_matches_scalar_library_conventions():
    """scalar.cpp:55-73 uses tanh-GELU, no bias, W_up [E,H,U], W_down [E,U,H];
    with those mapped in, the oracle's dispatch + combine must agree."""
    rng = np.random.default_rng(9)
    n, hid, u, e, k = 10, 8, 16, 4, 2
    x = torch.from_numpy(rng.standard_normal((n, hid)).astype(np.float32))
    wu = torch.from_numpy(rng.standard_normal((e, u, hid)).astype(np.float32) * 0.3)
    wd = torch.from_numpy(rng.standard_normal((e, hid, u)).astype(np.float32) * 0.3)
    ti = torch.from_numpy(rng.integers(0, e, (n, k)))
    ti[:, 1] = (ti[:, 0] + 1) % e
    tw = torch.from_numpy(rng.random((n, k)).astype(np.float32))
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(1, e), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(e * e, hid + 1), edge_gen_b=torch.zeros(e * e),
                       edge_value_w=torch.zeros(e, hid, hid), w_up=wu, w_down=wd)
    ours = B.expert_delta(x, ti, tw, w, act="gelu_tanh")
    rc, theirs = R.expert_grouped_gemm_f32(x.numpy(), ti.numpy(), tw.numpy(),
                                           wu.transpose(1, 2).numpy(), wd.transpose(1, 2).numpy())
    assert rc == 0
    np.testing.assert_allclose(ours.numpy(), theirs, rtol=1e-4, atol=1e-5)


@needs_ref
def test_epilogue_matches_scalar_library():
    rng = np.random.default_rng(10)
    n, hid = 12, 48
    h, d, x0 = (torch.from_numpy(rng.standard_normal((n, hid)).astype(np.float32)) for _ in range(3))
    g = torch.from_numpy(1 + 0.1 * rng.standard_normal(hid).astype(np.float32))
    b = torch.from_numpy(0.1 * rng.standard_normal(hid).astype(np.float32))
    w = B.BlockWeights(router_w=torch.zeros(1, hid), loop_bias=torch.zeros(1, 1), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(1, hid + 1), edge_gen_b=torch.zeros(1),
                       edge_value_w=torch.zeros(1, hid, hid), w_up=torch.zeros(1, 4, hid),
                       w_down=torch.zeros(1, hid, 4), ln_w=g, ln_b=b)
    ours = B.epilogue(h, d, x0, w)
    rc, theirs = R.loop_epilogue_f32(h.numpy(), d.numpy(), x0.numpy(), 0.5, 0.1, g.numpy(), b.numpy(), 1e-5)
    assert rc == 0
    np.testing.assert_allclose(ours.numpy(), theirs, rtol=1e-4, atol=1e-5)


# ------------------------------------------------------- closed forms ----
def _dense_delta(msg, ti, tw, w):
    """Dense all-expert mix (the construction of the reference's
    tests/test_sparse_experts_parity.py:41-50)."""
    up = torch.einsum("nh,euh->neu", msg, w.w_up)
    if w.b_up is not None:
        up = up + w.b_up.unsqueeze(0)
    if w.w_gate is not None:
        act = F.silu(torch.einsum("nh,euh->neu", msg, w.w_gate)) * up
    else:
        act = F.gelu(up)
    out = torch.einsum("neu,ehu->neh", act, w.w_down)
    if w.b_down is not None:
        out = out + w.b_down.unsqueeze(0)
    ew = torch.zeros(msg.shape[0], w.num_experts)
    ew.scatter_add_(-1, ti, tw)
    return (out * ew.unsqueeze(-1)).sum(1)


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_expert_delta_matches_dense_mix(act):
    g = torch.Generator().manual_seed(42)
    n, hid, e, k, u = 15, 32, 4, 2, 64
    msg = torch.randn(n, hid, generator=g)
    top_w, top_i = torch.randn(n, e, generator=g).softmax(-1).topk(k, dim=-1)
    top_w = top_w / top_w.sum(-1, keepdim=True)
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(1, e), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(e * e, hid + 1), edge_gen_b=torch.zeros(e * e),
                       edge_value_w=torch.zeros(e, hid, hid),
                       w_up=torch.randn(e, u, hid, generator=g), w_down=torch.randn(e, hid, u, generator=g),
                       b_up=None if act == "swiglu" else torch.randn(e, u, generator=g),
                       b_down=None if act == "swiglu" else torch.randn(e, hid, generator=g),
                       w_gate=torch.randn(e, u, hid, generator=g) if act == "swiglu" else None)
    dense = _dense_delta(msg, top_i, top_w, w)
    torch.testing.assert_close(B.expert_delta(msg, top_i, top_w, w), dense, rtol=1e-5, atol=1e-4)
    torch.testing.assert_close(B.expert_delta_planned(msg, top_i, top_w, w), dense, rtol=1e-5, atol=1e-4)


def test_swiglu_per_token_loop():
    """SwiGLU (not in the reference): closed form checked by a per-token loop."""
    g = torch.Generator().manual_seed(4)
    n, hid, e, k, u = 6, 8, 3, 2, 12
    msg = torch.randn(n, hid, generator=g)
    ti = torch.tensor([[0, 1], [1, 2], [2, 0], [0, 2], [1, 0], [2, 1]])
    tw = torch.rand(n, k, generator=g)
    wg, wu, wd = torch.randn(e, u, hid, generator=g), torch.randn(e, u, hid, generator=g), torch.randn(e, hid, u, generator=g)
    w = B.BlockWeights(router_w=torch.zeros(e, hid), loop_bias=torch.zeros(1, e), loop_emb=torch.zeros(1, 1),
                       edge_gen_w=torch.zeros(e * e, hid + 1), edge_gen_b=torch.zeros(e * e),
                       edge_value_w=torch.zeros(e, hid, hid), w_up=wu, w_down=wd, w_gate=wg)
    ref = torch.zeros(n, hid)
    for t in range(n):
        for s in range(k):
            ex = int(ti[t, s])
            a = msg[t] @ wg[ex].t()
            hidden = a / (1 + torch.exp(-a)) * (msg[t] @ wu[ex].t())
            ref[t] += tw[t, s] * (hidden @ wd[ex].t())
    torch.testing.assert_close(B.expert_delta(msg, ti, tw, w), ref, rtol=1e-5, atol=1e-5)


def test_planted_message_mistake_is_caught():
    """Applying router weights to sources (a plausible mistake: the legacy
    CSR kernel does, scalar.cpp:48) changes the message."""
    z, w, cfg = load_block("block_mid")
    hid = cfg["hidden_size"]
    h = torch.from_numpy(z["loop0/in"]).reshape(-1, hid)
    _, _, tw, ti = B.router(h, w, 0)
    ei, ew = B.edge_topm(B.edge_logits(h, w, 0), w.edges_per_expert)
    good = B.message_faithful(h, w, ti, ei, ew)
    coef_bad = torch.zeros(h.shape[0], w.num_experts)
    for s in range(ti.shape[1]):
        for j in range(ei.shape[-1]):
            d = ei[torch.arange(h.shape[0]), ti[:, s], j]
            coef_bad[torch.arange(h.shape[0]), d] += tw[:, s] * ew[torch.arange(h.shape[0]), ti[:, s], j]
    bad = B.message_grouped(h, w, coef_bad)
    assert (bad - good).abs().max() > 1e-2


# ------------------------------------------------------- early exit ----
def _exit_case():
    z, w, cfg = load_block("block_mid")
    hid = cfg["hidden_size"]
    h = torch.from_numpy(z["loop0/in"]).reshape(-1, hid)[:24]
    x0 = torch.randn(h.shape, generator=torch.Generator().manual_seed(11))
    return w, h, x0, cfg["num_loops"]


def test_exit_oracle_forced_exit_is_one_loop():
    """exit_head bias +20: every row leaves after loop 0 and keeps the
    loop-0 state (tests/test_early_exit_compaction.py:51-70)."""
    w, h, x0, r = _exit_case()
    one, _ = B.block_forward(h, x0, w, 0)
    out, loops, _ = B.block_loops_exit(h, x0, w, r, torch.zeros(h.shape[1]), 20.0, 0.85)
    assert torch.equal(out, one)
    assert (loops == 1).all()


def test_exit_oracle_no_exit_runs_all_loops():
    """exit_head bias -20: no row leaves; the result is the full loop run
    (tests/test_early_exit_compaction.py:73-82)."""
    w, h, x0, r = _exit_case()
    full = B.block_loops(h, x0, w, r)
    out, loops, _ = B.block_loops_exit(h, x0, w, r, torch.zeros(h.shape[1]), -20.0, 0.85)
    assert torch.equal(out, full)
    assert (loops == r).all()


def _per_token_exit(h, x0, w, r, ew, eb, thr):
    """Brute force: each row alone, loop by loop, until it exits."""
    outs, loops = [], []
    for t in range(h.shape[0]):
        ht, n = h[t:t + 1].float(), 0
        for li in range(r):
            ht, _ = B.block_forward(ht, x0[t:t + 1], w, li)
            n += 1
            if bool(torch.sigmoid(B.exit_logit(ht, ew, eb)) > thr):
                break
        outs.append(ht)
        loops.append(n)
    return torch.cat(outs), torch.tensor(loops)


def test_exit_oracle_matches_per_token_loop():
    """Partial exits (a random exit_head): the compacted batch equals each
    row run alone until its own exit (tests/test_early_exit_compaction.py:85-109
    checks the exited row against a single loop)."""
    w, h, x0, r = _exit_case()
    ew = torch.randn(h.shape[1], generator=torch.Generator().manual_seed(3)) * 0.5
    out, loops, margin = B.block_loops_exit(h, x0, w, r, ew, 0.0, 0.7)
    ref, ref_loops = _per_token_exit(h, x0, w, r, ew, 0.0, 0.7)
    assert len(set(loops.tolist())) >= 2, loops  # a mix of exit loops
    ok = margin > 1e-4
    assert torch.equal(loops[ok], ref_loops[ok])
    torch.testing.assert_close(out[ok], ref[ok], rtol=1e-5, atol=1e-5)


def test_planted_exit_mistake_is_caught():
    """Updating rows after they exit (dropping the compaction) differs from
    the per-row run."""
    w, h, x0, r = _exit_case()
    ew = torch.randn(h.shape[1], generator=torch.Generator().manual_seed(3)) * 0.5
    _, loops, _ = B.block_loops_exit(h, x0, w, r, ew, 0.0, 0.7)
    bad = B.block_loops(h, x0, w, r)  # every row runs every loop
    ref, _ = _per_token_exit(h, x0, w, r, ew, 0.0, 0.7)
    early = loops < r
    assert bool(early.any())
    assert (bad[early] - ref[early]).abs().max() > 1e-2


# ------------------------------------- sensitivity of the GPU checks ----
# The GPU parity tests compare the device's message and expert delta with the
# oracle (tests/_helpers.py: check_values) and the block outputs with a
# 1e-2 bound.  These CPU tests show, on the oracle, that (a) the bf16 storage
# the device uses stays well inside the value tolerances and (b) a missing
# message term, a missing expert, msg = 0 or delta = 0 fails them, at the
# shapes and weight scales the GPU tests run.
from _helpers import DELTA_TOL, MSG_TOL, oracle_weights, row_ratio  # noqa: E402

GPU_SMALL = dict(tokens=300, hidden_size=128, num_experts=8, top_k=2, edges_per_expert=3,
                 expert_ffn_size=256, num_loops=3, group_size=64, std="fan_in")


def _cpu_block(act, experts, **over):
    from spider_moe_amd.workloads import make_block
    spec = dict(GPU_SMALL)
    spec.update(over)
    wl = make_block("c1", device="cpu", expert_activation=act, experts=experts, **spec)
    n = wl.h.shape[0]
    return (wl.h.reshape(n, -1).float(), wl.x0.reshape(n, -1).float(), oracle_weights(wl.layer))


def _device_storage(h, w, aux):
    """The block's message and delta with the device's bf16 storage: each
    destination row c * W_edge[d] h rounded to bf16, their sum in ascending
    destination rounded to bf16; the FFN hidden activation and each expert's
    weighted output rounded to bf16, summed in ascending expert order."""
    n, hid = h.shape
    rb = B.round_bf16
    msg = torch.zeros(n, hid)
    for d in range(w.num_experts):
        c = aux.coef[:, d]
        rows = torch.nonzero(c != 0).flatten()
        if rows.numel():
            msg[rows] += rb(c[rows].unsqueeze(-1) * (h[rows] @ w.edge_value_w[d].t()))
    msg = rb(msg)
    delta = torch.zeros(n, hid)
    for e in range(w.num_experts):
        tw = (aux.top_w * (aux.top_i == e)).sum(-1)
        rows = torch.nonzero(tw > 0).flatten()
        if rows.numel():
            hid_act = B._expert_ffn(msg[rows], w, e, hidden_bf16=True)
            delta[rows] += rb(hid_act * tw[rows].unsqueeze(-1))
    return msg, delta


@pytest.mark.parametrize("act,experts", [("gelu", "bf16"), ("swiglu", "bf16"), ("swiglu", "fp8"),
                                         ("gelu", "int4")])
def test_value_tolerances_are_calibrated(act, experts):
    h, x0, w = _cpu_block(act, experts)
    _, aux = B.block_forward(h, x0, w, 0, out_bf16=True)
    msg, delta = _device_storage(h, w, aux)
    rm, rd = float(row_ratio(msg, aux.msg).max()), float(row_ratio(delta, aux.delta).max())
    assert rm < MSG_TOL / 3 and rd < DELTA_TOL / 2, (rm, rd)
    # planted mistakes: each token's last destination dropped from the message;
    # each token's second expert dropped from delta
    bad_msg = aux.msg.clone()
    for t in range(h.shape[0]):
        d = int(torch.nonzero(aux.coef[t]).flatten()[-1])
        bad_msg[t] -= aux.coef[t, d] * (h[t] @ w.edge_value_w[d].t())
    assert float(row_ratio(bad_msg, aux.msg).min()) > MSG_TOL
    tw = aux.top_w.clone()
    tw[:, 1] = 0.0
    bad_delta = B.expert_delta(aux.msg, aux.top_i, tw, w)
    assert float(row_ratio(bad_delta, aux.delta).min()) > DELTA_TOL
    assert float(row_ratio(torch.zeros_like(msg), aux.msg).min()) == 1.0


def _fails_bound(out, ref, tol=1e-2):
    return bool(((out - ref).abs() > tol + tol * ref.abs()).any())


@pytest.mark.parametrize("shape", ["gpu_small", "smoke"])
def test_output_bound_sees_message_and_delta(shape):
    """A block computed with delta = 0, or with msg = 0, fails the 1e-2
    output bound of the GPU block tests (so the bound checks the FFN and
    the message, not only the routing)."""
    if shape == "gpu_small":
        cases = [_cpu_block("gelu", "bf16"), _cpu_block("swiglu", "bf16")]
    else:  # the smoke: the c1 block (H 1024, std 0.02 weights), 64 tokens
        cases = [_cpu_block("swiglu", "bf16", tokens=64, hidden_size=1024, num_experts=16,
                            top_k=2, edges_per_expert=2, expert_ffn_size=2816, std=0.02)]
    for h, x0, w in cases:
        ref, aux = B.block_forward(h, x0, w, 0, out_bf16=True)
        no_delta = B.round_bf16(B.epilogue(h, torch.zeros_like(h), x0, w))
        assert _fails_bound(no_delta, ref)
        w0 = B.BlockWeights(**{**w.__dict__, "edge_value_w": torch.zeros_like(w.edge_value_w)})
        no_msg, _ = B.block_forward(h, x0, w0, 0, out_bf16=True)
        assert _fails_bound(no_msg, ref)
