"""Pins for oracle/dobu.py (the Dobu working-set policy) and the host logic
of the store, on the CPU (no GPU: the catalogue and the policy only)."""
import numpy as np
import torch
from torch import nn

from oracle import dobu as OD


def test_used_experts_merges_slots_and_drops_nonpositive():
    """expert_store.py:149-158: duplicates merge, a merged weight <= 0 (or
    an expert id outside [0, E)) is not used."""
    ti = np.array([[3, 1], [1, 1], [0, 7]])
    tw = np.array([[0.5, 0.5], [0.3, -0.3], [0.0, 1.0]], np.float32)
    assert OD.used_experts(ti, tw, 4) == [1, 3]


def test_lru_known_sequences():
    t = OD.LruTrace(2)
    t.step([0, 1])          # two misses
    t.step([1, 2])          # hit 1; miss 2 evicts 0
    assert (t.hits, t.misses, t.loads, t.hot) == (1, 3, 3, [1, 2])
    # more experts than the budget: 0 evicts 1, then 1 misses and evicts 2,
    # 2 evicts 0, 3 evicts 1 — four misses, no hit
    t.step([0, 1, 2, 3])
    assert t.hot == [2, 3] and t.misses == 7 and t.hits == 1
    z = OD.LruTrace(0)      # always stream
    z.step([1, 2])
    z.step([1])
    assert (z.hits, z.misses, z.loads, z.hot) == (0, 3, 3, [])


def test_lru_matches_a_brute_force_replay():
    """Independent restatement: the hot set is the last max distinct
    experts in touch order; a use is a hit iff that expert was in the hot
    set just before it."""
    rng = np.random.default_rng(5)
    for cap in (1, 2, 3, 5):
        t = OD.LruTrace(cap)
        touches = []
        hits = 0
        for _ in range(40):
            used = sorted(set(rng.integers(0, 8, rng.integers(1, 6)).tolist()))
            for e in used:
                order = []
                for x in reversed(touches):
                    if x not in order:
                        order.append(x)
                hits += e in order[:cap]
                touches.append(e)
            t.step(used)
        order = []
        for x in reversed(touches):
            if x not in order:
                order.append(x)
        assert t.hot == list(reversed(order[:cap]))
        assert t.hits == hits and t.misses == len(touches) - hits


def _experts(e=5, h=16, u=24, dtype=torch.float32):
    g = torch.Generator().manual_seed(3)
    mods = nn.ModuleList([nn.Sequential(nn.Linear(h, u), nn.GELU(), nn.Linear(u, h))
                          for _ in range(e)])
    with torch.no_grad():
        for p in mods.parameters():
            p.copy_(torch.randn(p.shape, generator=g))
    return mods.to(dtype)


def test_store_catalogue_and_stats_on_the_host():
    from spider_moe_amd.dobu import DobuConfig, ExpertChunkStore
    mods = _experts()
    st = ExpertChunkStore(mods, max_gpu_experts=3, pin_memory=False)
    assert len(st) == 5 and st.slots == 3
    assert torch.equal(st._chunks[2].w_up, mods[2][0].weight)
    assert torch.equal(st._chunks[4].b_down, mods[4][2].bias)
    s = st.stats()
    assert s["storage_bytes"] == 5 * (2 * 16 * 24 * 4 + 4 * (16 + 24))
    assert s["gpu_working_set_bytes"] == 0 and s["policy"] == "dobu_residency"
    d = DobuConfig(top_dobu=6).to_dict()
    assert d["top_dobu"] == 6 and "top_k" not in d  # tests/test_top_dobu.py:37-40
    bad = nn.ModuleList([nn.Sequential(nn.Linear(4, 8, bias=False), nn.GELU(), nn.Linear(8, 4))])
    try:
        ExpertChunkStore(bad, pin_memory=False)
        raise AssertionError("expected a ValueError")
    except ValueError:
        pass


def test_offloaded_layer_keeps_experts_on_the_host():
    """tests/test_expert_offload.py:34-42 and test_orbit_dobu.py:21-26:
    the expert modules stay on the CPU; top_k and top_dobu are separate."""
    from spider_moe_amd.config import ModelConfig
    from spider_moe_amd.dobu import DobuConfig, dobu_stats, enable_dobu
    from spider_moe_amd.model import SpiderWebLM
    cfg = ModelConfig(vocab_size=64, hidden_size=32, num_heads=4, num_experts=8, top_k=2,
                      edges_per_expert=2, num_loops=2, num_prelude_layers=1, num_coda_layers=1,
                      expert_ffn_size=64, loop_embed_size=8, max_seq_len=32, use_rope=True,
                      offload_experts=True, offload_max_gpu_experts=2)
    model = SpiderWebLM(cfg).eval()
    model.to("cpu")
    for ex in model.recurrent.experts:
        assert next(ex.parameters()).device.type == "cpu"
    assert model.recurrent._expert_store.stats()["num_experts"] == 8
    cfg2 = ModelConfig(vocab_size=64, hidden_size=32, num_heads=4, num_experts=8, top_k=3,
                       edges_per_expert=2, num_loops=2, num_prelude_layers=1, num_coda_layers=1,
                       expert_ffn_size=64, loop_embed_size=8, max_seq_len=32, use_rope=True)
    m2 = SpiderWebLM(cfg2).eval()
    enable_dobu(m2, DobuConfig(top_dobu=5))
    assert m2.cfg.top_k == 3 and m2.recurrent.top_k == 3
    assert m2.recurrent.top_dobu == 5 and m2.recurrent._expert_store.max_gpu_experts == 5
    st = dobu_stats(m2)
    assert st["top_k"] == 3 and st["top_dobu"] == 5
    assert st["top_k_role"] == "router_experts_per_token"
    assert st["top_dobu_role"] == "gpu_chunk_residency_lru"
