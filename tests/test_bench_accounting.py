"""bench.py's contract on the CPU: the single-GPU refusal and the
algorithmic work its roofline divides by (bytes and flops per launch of the
expert GEMMs, per step of the block), checked against figures worked out by
hand for the benchmark shapes."""
import os
import subprocess
import sys
from types import SimpleNamespace

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _layer(h, u, act, fmt, group=128, sdt=torch.float16):
    q = SimpleNamespace(group_size=group, scales=torch.zeros(1, dtype=sdt))
    return SimpleNamespace(hidden_size=h, expert_ffn_size=u, expert_activation=act,
                           expert_format=fmt, _int4_w_up=q, _int4_w_down=q,
                           num_experts=16, top_k=2, loop_embed_size=0)


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=60)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


def test_decode_fp8_gemm_bytes():
    # c2: H 1024, U 2816, SwiGLU, fp8 weights with fp32 per-channel scales,
    # 16 experts touched by 128 (token, expert) rows.
    layer = _layer(1024, 2816, "swiglu", "fp8")
    # up: 5632 x 1024 codes + 5632 scales (4 B) per expert; rows in (H bf16) and out (U bf16)
    assert bench.up_gemm_bytes(layer, 128, 16) == 16 * (5632 * 1024 + 4 * 5632) + 128 * 2048 + 128 * 5632
    assert bench.up_gemm_bytes(layer, 128, 16) == 93_618_176
    # down: 1024 x 2816 codes + 1024 scales per expert; rows in (U) and out (H)
    assert bench.down_gemm_bytes(layer, 128, 16) == 47_185_920


def test_int4_gemm_bytes():
    # c4: H 2048, U 1408, GELU (fp32 biases), int4 group 128 with fp16 scales,
    # 64 experts touched by 4352 rows.
    layer = _layer(2048, 1408, "gelu", "int4")
    per_expert = 1408 * 2048 // 2 + 2 * 1408 * 16 + 4 * 1408
    assert per_expert == 1_492_480
    assert bench.up_gemm_bytes(layer, 4352, 64) == 64 * per_expert + 4352 * (4096 + 2816)
    assert bench.up_gemm_bytes(layer, 4352, 64) == 125_599_744


def test_prefill_gemm_flops():
    # c1 up GEMM: 32768 (token, expert) rows, SwiGLU: 4 H U flops per row
    layer = _layer(1024, 2816, "swiglu", "bf16")
    acc = [dict(s_rows=32768, e_touched=16, d_rows=0, d_touched=0)]
    f, _ = bench.gemm_work(layer, "up_gemm", acc)
    assert f == 377_957_122_048  # 3.78e11, the bench line's work_per_launch
    f, _ = bench.gemm_work(layer, "down_gemm", acc)
    assert f == 2 * 1024 * 2816 * 32768
    acc = [dict(s_rows=0, e_touched=0, d_rows=1000, d_touched=16)]
    f, b = bench.gemm_work(layer, "edge_gemm", acc)
    assert f == 2 * 1024 * 1024 * 1000
    assert b == 16 * 2 * 1024 * 1024 + 1000 * 1024 * 4


def test_block_flops_per_step():
    # per token and loop: 2HE (router) + 2(H+L)Ek (edge logits of the k
    # selected sources) + 2H^2 |D_t| + 6HU |S_t| (SwiGLU up and down)
    layer = _layer(1024, 2816, "swiglu", "bf16")
    n = 4
    acc = [dict(s_rows=8, e_touched=5, d_rows=11, d_touched=7)]
    f, _ = bench.block_work(layer, n, acc)
    assert f == 4 * 2 * 1024 * 16 + 4 * 2 * 1024 * 16 * 2 + 2 * 1024 ** 2 * 11 + 6 * 1024 * 2816 * 8
