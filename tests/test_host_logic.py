"""CPU checks of the host-side package: weight formats (against the oracle),
the SwiGLU block interleave, drop-in parameter names, workloads, and that
nothing falls back to the CPU."""
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import quant as Q


def test_int4_packing_matches_oracle_and_reference():
    from spider_moe_amd.quant import dequantize_int4, quantize_int4
    z = np.load(os.path.join(GOLDEN, "quant_int4.npz"))
    w = torch.from_numpy(z["w"])
    for gs in (32, 64, 128, 48):
        q = quantize_int4(w, gs)
        assert np.array_equal(q.packed.numpy(), z[f"g{gs}/packed"])
        assert np.array_equal(q.scales.numpy(), z[f"g{gs}/scales"])
        assert np.array_equal(dequantize_int4(q.packed, q.scales, q.shape, q.group_size).numpy(),
                              z[f"g{gs}/deq"])
    q16 = quantize_int4(w, 128, torch.float16)
    assert np.array_equal(q16.packed.numpy(), z["g128/packed"])
    assert q16.scales.dtype == torch.float16


def test_fp8_per_channel_matches_oracle():
    from spider_moe_amd.quant import quantize_fp8_per_channel
    w = torch.randn(3, 40, 64, generator=torch.Generator().manual_seed(0)) * 0.02
    codes, scale = quantize_fp8_per_channel(w)
    oc, os_ = Q.fp8_quantize_per_channel(w.numpy())
    assert np.array_equal(codes.view(torch.uint8).numpy(), oc)
    assert np.array_equal(scale.numpy(), os_)


def test_swiglu_interleave_layout():
    from spider_moe_amd.quant import interleave_gate_up
    u, x = 96, 3
    gate = torch.arange(u * x).view(1, u, x).float()
    up = -torch.arange(u * x).view(1, u, x).float() - 1
    out = interleave_gate_up(gate, up)[0]
    for j in range(u // 32):
        assert torch.equal(out[64 * j: 64 * j + 32], gate[0, 32 * j: 32 * j + 32])
        assert torch.equal(out[64 * j + 32: 64 * j + 64], up[0, 32 * j: 32 * j + 32])


def test_state_dict_keys_match_reference_layer():
    from spider_moe_amd import ModelConfig, SpiderMoELayer
    z = np.load(os.path.join(GOLDEN, "block_small.npz"))
    ref_keys = {k[6:] for k in z.files if k.startswith("param/")}
    cfg = ModelConfig(vocab_size=64, hidden_size=32, num_heads=4, num_experts=4, top_k=2,
                      edges_per_expert=2, num_loops=2, expert_ffn_size=64, loop_embed_size=8)
    layer = SpiderMoELayer(cfg)
    assert set(layer.state_dict().keys()) == ref_keys
    sd = {k[6:]: torch.from_numpy(z[k]) for k in z.files if k.startswith("param/")}
    layer.load_state_dict(sd)


def test_lm_state_dict_keys_match_reference():
    from spider_moe_amd import ModelConfig, SpiderWebLM
    z = np.load(os.path.join(GOLDEN, "lm_c0.npz"))
    ref_keys = {k[6:] for k in z.files if k.startswith("param/")}
    c = {k[4:]: int(z[k]) for k in z.files if k.startswith("cfg/")}
    model = SpiderWebLM(ModelConfig(**c))
    ours = set(model.state_dict().keys()) - {"position_embedding.weight", "lm_head.weight"}
    assert ours == ref_keys


def test_no_cpu_fallback():
    from spider_moe_amd import ModelConfig, SpiderMoELayer, sparse_expert_delta
    cfg = ModelConfig(hidden_size=32, num_heads=4, num_experts=4, top_k=2, edges_per_expert=2,
                      num_loops=2, expert_ffn_size=64, loop_embed_size=8)
    layer = SpiderMoELayer(cfg).eval()
    h = torch.randn(1, 4, 32)
    with pytest.raises(RuntimeError, match="GPU"):
        with torch.no_grad():
            layer(h, h, 0)
    with pytest.raises(RuntimeError, match="GPU"):
        sparse_expert_delta(h, torch.zeros(1, 4, 2, dtype=torch.long), torch.ones(1, 4, 2),
                            torch.zeros(4, 64, 32), torch.zeros(4, 64), torch.zeros(4, 32, 64),
                            torch.zeros(4, 32), num_experts=4, top_k=2)


def test_config_validation_and_unsupported_features():
    from spider_moe_amd import ModelConfig, SpiderMoELayer
    with pytest.raises(ValueError):
        ModelConfig(num_experts=2, top_k=3).validate()
    with pytest.raises(ValueError):
        ModelConfig(expert_activation="relu").validate()
    with pytest.raises(NotImplementedError):
        SpiderMoELayer(ModelConfig(use_lumen=True))
    with pytest.raises(ValueError):  # Dobu holds Linear + GELU + Linear experts
        SpiderMoELayer(ModelConfig(offload_experts=True, expert_activation="swiglu"))


def test_zipf_bias_forces_empty_experts():
    from spider_moe_amd.workloads import zipf_loop_bias
    b = zipf_loop_bias(4, 32, 1.2, 4, torch.Generator().manual_seed(0))
    assert b.shape == (4, 32)
    assert int((b[0] == -1e4).sum()) == 4
    assert torch.equal(b[0], b[3])
    live = b[0][b[0] > -1e3]
    assert sorted((-live / 1.2).exp().round().long().tolist()) == list(range(1, 29))
    b0 = zipf_loop_bias(2, 8, 1.2, 0, torch.Generator().manual_seed(0))
    assert bool((b0 > -1e3).all())
