"""GPU parity of Orbit Dobu expert offload (ExpertChunkStore.sparse_delta,
SpiderMoELayer / SpiderWebLM with offload_experts) against the oracle:
the FFN values of oracle.block.expert_delta, the working-set bookkeeping of
oracle.dobu.LruTrace, and the resident path on the same weights.

Tolerances: fp32 experts run the fp32 GEMM path, so the store's delta
matches the oracle at rtol 1e-4 and the resident path (same kernels, slot
order instead of expert order in the combine) at 1e-5; bf16 experts use
the block's message / delta ratio bounds (tests/_helpers.py)."""
import numpy as np
import pytest
import torch

from oracle import block as B
from oracle import dobu as OD
from _helpers import DELTA_TOL, row_ratio

pytestmark = pytest.mark.gpu

dev = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def _experts(e, h, u, dtype, seed):
    from torch import nn
    g = torch.Generator().manual_seed(seed)
    mods = nn.ModuleList([nn.Sequential(nn.Linear(h, u), nn.GELU(), nn.Linear(u, h))
                          for _ in range(e)])
    with torch.no_grad():
        for p in mods.parameters():
            p.copy_(torch.randn(p.shape, generator=g) / (p.shape[-1] ** 0.5))
    return mods.to(dtype)


def _oracle_weights(mods):
    """The expert part of oracle.block.BlockWeights (the rest unused here)."""
    e = len(mods)
    h = mods[0][0].weight.shape[1]
    z = torch.zeros
    return B.BlockWeights(
        router_w=z(e, h), loop_bias=z(1, e), loop_emb=z(1, 1), edge_gen_w=z(e * e, h + 1),
        edge_gen_b=z(e * e), edge_value_w=z(e, 1, 1),
        w_up=torch.stack([m[0].weight.detach().float().cpu() for m in mods]),
        w_down=torch.stack([m[2].weight.detach().float().cpu() for m in mods]),
        b_up=torch.stack([m[0].bias.detach().float().cpu() for m in mods]),
        b_down=torch.stack([m[2].bias.detach().float().cpu() for m in mods]))


def worst(got, ref):
    return row_ratio(got.float().cpu().reshape(ref.shape[0], -1),
                     ref.float().cpu().reshape(ref.shape[0], -1)).max().item()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("top_dobu", [0, 2, 5, 16])
def test_store_delta_and_working_set(dtype, top_dobu):
    """Three steps through one store: every delta against the oracle's
    sparse_expert_delta, the hits / misses / loads / hot set against the
    reference's LRU restated, and fp32 deltas against the resident kernels."""
    from spider_moe_amd.dobu import ExpertChunkStore
    from spider_moe_amd.sparse_experts import sparse_expert_delta
    e, h, u, k = 12, 128, 256, 3
    say("dobu store", dtype, top_dobu)
    mods = _experts(e, h, u, dtype, 7)
    store = ExpertChunkStore(mods, max_gpu_experts=top_dobu)
    trace = OD.LruTrace(top_dobu)
    ow = _oracle_weights(mods)
    g = torch.Generator().manual_seed(11)
    for step, n in enumerate((300, 40, 777)):
        msg = torch.randn(1, n, h, generator=g).to(dtype)
        ti = torch.randint(0, e if step != 1 else 4, (1, n, k), generator=g)
        ti[0, 0] = torch.tensor([2, 2, 1])  # a duplicate slot merges
        tw = torch.rand(1, n, k, generator=g)
        tw[0, 1, 0] = 0.0
        got = store.sparse_delta(msg.to(dev), ti.to(dev), tw.to(dev), k)
        assert got.shape == msg.shape and got.dtype == dtype
        trace.step(OD.used_experts(ti.numpy(), tw.numpy(), e))
        st = store.stats()
        assert (st["hits"], st["misses"], st["loads"]) == (trace.hits, trace.misses, trace.loads)
        assert st["gpu_hot_experts"] == trace.hot
        want = B.expert_delta(msg[0].float(), ti[0], tw[0], ow, act="gelu")
        gf = got[0].float().cpu()
        if dtype == torch.float32:
            assert torch.allclose(gf, want, rtol=1e-4, atol=1e-4)
            res = sparse_expert_delta(
                msg.to(dev), ti.to(dev), tw.to(dev), ow.w_up.to(dev), ow.b_up.to(dev),
                ow.w_down.to(dev), ow.b_down.to(dev), num_experts=e, top_k=k)
            assert torch.allclose(got, res, rtol=1e-5, atol=1e-5)
        else:
            assert worst(gf, want) < DELTA_TOL
    if top_dobu > 0:
        assert len(store.stats()["gpu_hot_experts"]) <= top_dobu
    store.release_gpu()
    assert store.stats()["gpu_hot_experts"] == []


def _lm_cfg(offload, top_k=2, top_dobu=2):
    from spider_moe_amd.config import ModelConfig
    return ModelConfig(vocab_size=64, hidden_size=32, num_heads=4, num_experts=8, top_k=top_k,
                       edges_per_expert=2, num_loops=2, num_prelude_layers=1,
                       num_coda_layers=1, expert_ffn_size=64, loop_embed_size=8,
                       max_seq_len=32, dropout=0.0, expert_parallel=False, use_rope=True,
                       offload_experts=offload, offload_max_gpu_experts=top_dobu).validate()


def test_offloaded_lm_matches_the_resident_lm():
    """tests/test_expert_offload.py:45-70 and test_orbit_dobu.py:48-56:
    same weights, offloaded vs resident experts -> logits within 1e-4."""
    from spider_moe_amd.dobu import DobuConfig, dobu_stats, enable_dobu
    from spider_moe_amd.model import SpiderWebLM
    say("offloaded lm")
    torch.manual_seed(0)
    a = SpiderWebLM(_lm_cfg(False)).eval()
    torch.manual_seed(0)
    b = SpiderWebLM(_lm_cfg(False)).eval()
    b.load_state_dict(a.state_dict())
    a, b = a.to(dev), b.to(dev)
    store = enable_dobu(b, DobuConfig(top_dobu=4))
    assert all(next(ex.parameters()).device.type == "cpu" for ex in b.recurrent.experts)
    x = torch.randint(0, 64, (2, 5), generator=torch.Generator().manual_seed(1)).to(dev)
    with torch.no_grad():
        la, lb = a(x)["logits"], b(x)["logits"]
        ea, eb = a(x, early_exit=True), b(x, early_exit=True)
    assert torch.allclose(la, lb, rtol=1e-4, atol=1e-4)
    assert torch.allclose(ea["logits"], eb["logits"], rtol=1e-4, atol=1e-4)
    assert ea["loops_used"] == eb["loops_used"]
    st = dobu_stats(b)
    assert st["loads"] >= 1 and len(st["gpu_hot_experts"]) <= 4 and store is b.recurrent._expert_store
    # top_dobu below top_k is allowed (tests/test_top_dobu.py:43-50)
    m = SpiderWebLM(_lm_cfg(False, top_k=3)).eval().to(dev)
    enable_dobu(m, DobuConfig(top_dobu=2))
    with torch.no_grad():
        y = m(x)["logits"]
    assert y.shape == (2, 5, 64) and torch.isfinite(y).all()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_offloaded_block_matches_resident_block(dtype):
    """A larger block (H 256, E 16, 3 loops): the offloaded layer's output
    against the resident layer (same weights), the loop-by-loop working set
    against the LRU oracle fed the routing the layer reports, and a weight
    update that must reach the catalogue."""
    from spider_moe_amd.workloads import make_block
    say("offloaded block", dtype)
    kw = dict(tokens=400, hidden_size=256, num_experts=16, top_k=2, edges_per_expert=3,
              expert_ffn_size=512, num_loops=3, dtype=dtype, experts=dtype, std="fan_in",
              expert_activation="gelu")
    res = make_block("c1", **kw)
    off = make_block("c1", **kw)
    store = off.layer.enable_offload(top_dobu=5)
    assert all(p.device.type == "cpu" for p in off.layer.experts.parameters())
    off.layer.to(dev)  # stays offloaded
    assert all(p.device.type == "cpu" for p in off.layer.experts.parameters())
    trace = OD.LruTrace(5)
    h = res.h
    tol = 1e-4 if dtype == "f32" else 2e-2
    with torch.no_grad():
        for r in range(3):  # each loop from the same input (no routing drift)
            h_r = res.layer(h, res.x0, r)
            h_o = off.layer(h, off.x0, r)
            rt = off.layer.last_routing()
            trace.step(OD.used_experts(rt["top_idx"].cpu().numpy(), rt["top_w"].cpu().numpy(), 16))
            assert worst(h_o, h_r) < tol
            h = h_r
        st = store.stats()
        assert (st["hits"], st["misses"], st["loads"]) == (trace.hits, trace.misses, trace.loads)
        assert st["gpu_hot_experts"] == trace.hot
        # a changed expert weight reaches the catalogue on the next call
        for lay in (res.layer, off.layer):
            lay.experts[3][2].bias.data.add_(0.5)
        a = res.layer(res.h, res.x0, 0)
        b = off.layer(off.h, off.x0, 0)
        assert worst(b, a) < tol
        assert all(p.device.type == "cpu" for p in off.layer.experts.parameters())
        if dtype == "f32":  # the exit gate over 3 loops (bf16 rounding would let routing drift)
            ea, _, la = res.layer.forward_loops_exit(res.h, res.x0, 0.6)
            eb, _, lb = off.layer.forward_loops_exit(off.h, off.x0, 0.6)
            assert (la == lb).float().mean().item() > 0.98
            ra = row_ratio(eb.float().cpu().reshape(-1, 256), ea.float().cpu().reshape(-1, 256))
            assert (ra < tol).float().mean().item() > 0.98
