"""GPU parity of the individual stages (router, dispatch plan, expert FFN in
every weight format) against the oracle, through the C ABI."""
import ctypes
import os

import numpy as np
import pytest
import torch

from conftest import GOLDEN
from oracle import block as B
from oracle import plan as P
from oracle import quant as Q

pytestmark = pytest.mark.gpu

dev = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def nat():
    from spider_moe_amd import _native
    _native.lib()
    return _native


# ------------------------------------------------------------- router ----
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("e,k", [(4, 2), (16, 2), (32, 4), (64, 2), (64, 8), (100, 3), (200, 16),
                                 (256, 4)])
@pytest.mark.parametrize("n", [1000, 40])  # 40 tokens: the decode (weight-streaming) GEMM
def test_router_topk_matches_oracle(dtype, e, k, n):
    """E > 64: one wave per token, up to four experts per lane."""
    n8 = nat()
    h = 256
    say("router", dtype, e, k, n)
    g = torch.Generator().manual_seed(e * 10 + k)
    x = torch.randn(n, h, generator=g).to(dtype)
    w = (torch.randn(e, h, generator=g) * 0.1).to(dtype)
    lb = torch.randn(e, generator=g) * 0.5
    xd, wd, lbd = x.to(dev), w.to(dev), lb.to(dev)
    logits = torch.empty(n, e, device=dev)
    tw = torch.empty(n, k, device=dev)
    ti = torch.empty(n, k, dtype=torch.int32, device=dev)
    need = n8.lib().smoe_router_workspace_bytes(n, e)
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    n8.check(n8.lib().smoe_router_topk(xd.data_ptr(), n8.dtype_code(dtype), n, h, wd.data_ptr(),
                                       lbd.data_ptr(), e, k, logits.data_ptr(), tw.data_ptr(),
                                       ti.data_ptr(), ws.data_ptr(), need,
                                       n8.stream_of(torch.device(dev))), "router")
    torch.cuda.synchronize()
    ow = B.BlockWeights(router_w=w.float(), loop_bias=lb.view(1, -1), loop_emb=torch.zeros(1, 1),
                        edge_gen_w=torch.zeros(e * e, h + 1), edge_gen_b=torch.zeros(e * e),
                        edge_value_w=torch.zeros(1, 1, 1), w_up=torch.zeros(1, 1, 1),
                        w_down=torch.zeros(1, 1, 1), top_k=k)
    ol, _, otw, oti = B.router(x.float(), ow, 0)
    np.testing.assert_allclose(logits.cpu().numpy(), ol.numpy(), rtol=1e-5, atol=2e-5)
    gap = B._kth_gap(ol, k)
    ok = gap >= 1e-6
    assert (ti.cpu().long()[ok] == oti[ok]).all(), "top-k indices differ on non-tie tokens"
    np.testing.assert_allclose(tw.cpu()[ok].numpy(), otw[ok].numpy(), rtol=2e-5, atol=1e-6)
    assert ok.float().mean() > 0.98


# ------------------------------------------------------- dispatch plan ----
@pytest.mark.parametrize("n,k,e", [(0, 2, 4), (1, 1, 1), (100, 2, 4), (777, 3, 16),
                                   (5000, 2, 16), (20000, 4, 32), (3000, 8, 64),
                                   (4000, 12, 64), (70000, 20, 200), (300, 40, 256)])
def test_dispatch_plan_bit_exact(n, k, e):
    from spider_moe_amd.dispatch import plan_tensors
    say("plan", n, k, e)
    rng = np.random.default_rng(n + k + e)
    idx = rng.integers(-1, e + 1, (n, k)).astype(np.int64)  # includes out-of-range ids
    w = rng.random((n, k)).astype(np.float32)
    if n:
        w[rng.random((n, k)) < 0.1] = 0.0
        w[rng.random((n, k)) < 0.05] *= -1.0
        idx[: n // 10, :] = idx[: n // 10, :1]                  # duplicates
    counts, offsets, rows, roww, tokrow = plan_tensors(torch.from_numpy(idx).to(dev),
                                                       torch.from_numpy(w).to(dev), e)
    torch.cuda.synchronize()
    _, ocnt, operm, opw, orow_e = P.dispatch_plan(idx, w, e)
    assert counts.cpu().numpy().tolist() == ocnt.tolist()
    off = offsets.cpu().numpy()
    assert off[0] == 0 and off[-1] == len(operm)
    assert rows[: off[-1]].cpu().numpy().tolist() == operm.tolist()
    assert np.array_equal(roww[: off[-1]].cpu().numpy(), opw)
    # tok_row points back at the token's own rows, ascending expert order
    tr = tokrow.cpu().numpy()
    r_np = rows.cpu().numpy()
    for t in range(min(n, 500)):
        got = [r for r in tr[t] if r >= 0]
        assert all(r_np[r] == t for r in got)
        assert got == sorted(got)


def test_dispatch_plan_reference_known_answer():
    from spider_moe_amd.dispatch import build_dispatch_plan
    say("plan known answer")
    ti = torch.tensor([[[0, 1], [1, 2]]], device=dev)
    tw = torch.tensor([[[0.7, 0.3], [0.6, 0.4]]], device=dev)
    plan = build_dispatch_plan(ti, tw, num_experts=4, local_only=False)
    assert {a.expert_id for a in plan.assignments} == {0, 1, 2}
    assert plan.tokens_for(1).token_index.numel() == 2


# ------------------------------------------------------- expert delta ----
def _delta_case(n, h, u, e, k, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    msg = torch.randn(n, h, generator=g)
    idx = torch.randint(0, e, (n, k), generator=g)
    w = torch.rand(n, k, generator=g)
    wu = torch.randn(e, u, h, generator=g) * scale
    bu = torch.randn(e, u, generator=g) * 0.1
    wd = torch.randn(e, h, u, generator=g) * scale
    bd = torch.randn(e, h, generator=g) * 0.1
    return msg, idx, w, wu, bu, wd, bd


def _oracle_delta(msg, idx, w, wu, bu, wd, bd, w_gate=None, hidden_bf16=False):
    e, _, h = wu.shape
    ow = B.BlockWeights(router_w=torch.zeros(e, h), loop_bias=torch.zeros(1, e), loop_emb=torch.zeros(1, 1),
                        edge_gen_w=torch.zeros(e * e, h + 1), edge_gen_b=torch.zeros(e * e),
                        edge_value_w=torch.zeros(e, 1, 1), w_up=wu, w_down=wd, b_up=bu, b_down=bd,
                        w_gate=w_gate)
    return B.expert_delta(msg, idx, w, ow, hidden_bf16=hidden_bf16)


def test_sparse_expert_delta_golden_f32():
    from spider_moe_amd import sparse_expert_delta
    say("sparse delta golden")
    z = np.load(os.path.join(GOLDEN, "sparse_delta.npz"))
    t = {k: torch.from_numpy(z[k]).to(dev) for k in z.files}
    e = t["w_up"].shape[0]
    # the reference's own case as given: H 16, U 24 (K tails of the GEMMs masked)
    d = sparse_expert_delta(t["msg"], t["idx"], t["w"], t["w_up"], t["b_up"], t["w_down"],
                            t["b_down"], num_experts=e, top_k=t["idx"].shape[-1],
                            expert_parallel=False)
    torch.testing.assert_close(d.cpu(), t["delta"].cpu(), rtol=1e-5, atol=1e-5)
    # bf16 at the same odd shape runs the SIMT GEMM (K = 16 and 24)
    bf = torch.bfloat16
    d16 = sparse_expert_delta(t["msg"].to(bf), t["idx"], t["w"], t["w_up"].to(bf), t["b_up"],
                              t["w_down"].to(bf), t["b_down"], num_experts=e,
                              top_k=t["idx"].shape[-1])
    ref16 = _oracle_delta(t["msg"].to(bf).float().cpu().reshape(-1, 16),
                          t["idx"].cpu().reshape(-1, 3), t["w"].cpu().reshape(-1, 3),
                          t["w_up"].to(bf).float().cpu(), t["b_up"].cpu(),
                          t["w_down"].to(bf).float().cpu(), t["b_down"].cpu())
    torch.testing.assert_close(d16.float().cpu().reshape(-1, 16), ref16, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,h,u,e,k", [(300, 40, 56, 6, 2), (77, 24, 100, 100, 3),
                                       (500, 64, 96, 256, 4), (33, 200, 72, 13, 2)])
def test_sparse_expert_delta_any_shape(dtype, n, h, u, e, k):
    """H and U off the MFMA grid (K tails masked in the SIMT kernel, any
    row width in the combine) and E up to 256, against the oracle."""
    from spider_moe_amd import sparse_expert_delta
    say("sparse delta any shape", dtype, n, h, u, e, k)
    msg, idx, w, wu, bu, wd, bd = _delta_case(n, h, u, e, k, 17)
    wu, wd = wu.to(dtype).float(), wd.to(dtype).float()
    ref = _oracle_delta(msg.to(dtype).float(), idx, w, wu, bu, wd, bd)
    got = sparse_expert_delta(msg.to(dev, dtype).view(1, n, h), idx.to(dev).view(1, n, k),
                              w.to(dev).view(1, n, k), wu.to(dev, dtype), bu.to(dev),
                              wd.to(dev, dtype), bd.to(dev), num_experts=e, top_k=k)
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    torch.testing.assert_close(got.float().cpu().view(n, h), ref, rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_sparse_expert_delta_matches_oracle(dtype):
    from spider_moe_amd import sparse_expert_delta
    say("sparse delta", dtype)
    msg, idx, w, wu, bu, wd, bd = _delta_case(257, 128, 192, 6, 3, 5)
    idx[:20, 1] = idx[:20, 0]        # duplicates
    w[20:30, 0] = 0.0                # zero weights
    wu, wd = wu.to(dtype).float(), wd.to(dtype).float()
    ref = _oracle_delta(msg.to(dtype).float(), idx, w, wu, bu, wd, bd)
    got = sparse_expert_delta(msg.to(dev, dtype).view(1, 257, 128), idx.to(dev).view(1, 257, 3),
                              w.to(dev).view(1, 257, 3), wu.to(dev, dtype), bu.to(dev),
                              wd.to(dev, dtype), bd.to(dev), num_experts=6, top_k=3)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    torch.testing.assert_close(got.float().cpu().view(257, 128), ref, rtol=tol, atol=tol)


def _experts_struct(n8, fmt, act, e, h, u, w_up, w_down, s_up=None, s_down=None, b_up=None,
                    b_down=None, group=0, scale_dtype=0):
    ex = n8.SmoeExperts()
    ex.format, ex.act, ex.E, ex.H, ex.U = fmt, act, e, h, u
    ex.group_size, ex.scale_dtype = group, scale_dtype
    ex.w_up, ex.w_down = w_up.data_ptr(), w_down.data_ptr()
    ex.s_up = s_up.data_ptr() if s_up is not None else None
    ex.s_down = s_down.data_ptr() if s_down is not None else None
    ex.b_up = b_up.data_ptr() if b_up is not None else None
    ex.b_down = b_down.data_ptr() if b_down is not None else None
    return ex


def _tiles(n8, w, code=None):
    """bf16 (or fp8 codes, code FP8_E4M3) [G,N,K] -> the weight tile layout
    through smoe_pack_weight_tiles."""
    out = torch.empty_like(w)
    code = n8.BF16 if code is None else code
    n8.check(n8.lib().smoe_pack_weight_tiles(w.data_ptr(), code, w.shape[0], w.shape[1],
                                             w.shape[2], out.data_ptr(),
                                             n8.stream_of(torch.device(dev))),
             "pack_weight_tiles")
    torch.cuda.synchronize()
    return out


def test_pack_weight_tiles_layout():
    """out[(((g*T + t)*S + s)*2 + h)*64 + l][e] = w[g][16t + l%16][64s + 32h + 8(l/16) + e]
    (include/smoe.h), checked element by element on a small case and as one
    permutation of the whole tensor."""
    n8 = nat()
    say("pack weight tiles")
    g_, n_, k_ = 3, 48, 192
    w = torch.randn(g_, n_, k_, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(dev)
    got = _tiles(n8, w).cpu().view(-1, 8)
    wc = w.cpu()
    t_, s_ = n_ // 16, k_ // 64
    rng = np.random.default_rng(9)
    for _ in range(200):
        g, t, s, h, l = (int(rng.integers(0, x)) for x in (g_, t_, s_, 2, 64))
        f = (((g * t_ + t) * s_ + s) * 2 + h) * 64 + l
        ref = wc[g, 16 * t + l % 16, 64 * s + 32 * h + 8 * (l // 16): 64 * s + 32 * h + 8 * (l // 16) + 8]
        assert torch.equal(got[f], ref), (g, t, s, h, l)
    perm = wc.view(g_, t_, 16, s_, 2, 4, 8).permute(0, 1, 3, 4, 5, 2, 6).reshape(-1, 8)
    assert torch.equal(got, perm)


def test_pack_weight_tiles_layout_fp8():
    """fp8 codes: out[((g*T + t)*S + s)*64 + l][e] = w[g][16t + l%16][64s + 16(l/16) + e]
    (include/smoe.h), element by element and as one permutation; int4 and
    f32 are refused."""
    n8 = nat()
    say("pack weight tiles fp8")
    g_, n_, k_ = 2, 32, 320
    w = torch.randint(0, 256, (g_, n_, k_), dtype=torch.uint8,
                      generator=torch.Generator().manual_seed(6)).to(dev)
    got = _tiles(n8, w, n8.FP8_E4M3).cpu().view(-1, 16)
    wc = w.cpu()
    t_, s_ = n_ // 16, k_ // 64
    rng = np.random.default_rng(10)
    for _ in range(200):
        g, t, s, l = (int(rng.integers(0, x)) for x in (g_, t_, s_, 64))
        f = ((g * t_ + t) * s_ + s) * 64 + l
        ref = wc[g, 16 * t + l % 16, 64 * s + 16 * (l // 16): 64 * s + 16 * (l // 16) + 16]
        assert torch.equal(got[f], ref), (g, t, s, l)
    perm = wc.view(g_, t_, 16, s_, 4, 16).permute(0, 1, 3, 4, 2, 5).reshape(-1, 16)
    assert torch.equal(got, perm)
    out = torch.empty_like(w)
    for code in (n8.INT4, n8.F32):
        rc = n8.lib().smoe_pack_weight_tiles(w.data_ptr(), code, g_, n_, k_, out.data_ptr(),
                                             n8.stream_of(torch.device(dev)))
        assert rc == -2


def _run_delta(n8, ex, msg_bf16, idx, w):
    n, k = idx.shape
    h = msg_bf16.shape[1]
    out = torch.empty(n, h, device=dev)
    need = n8.lib().smoe_expert_delta_workspace_bytes(ctypes.byref(ex), n, k)
    assert need > 0, n8.lib().smoe_last_error()
    ws = torch.empty(need, dtype=torch.uint8, device=dev)
    n8.check(n8.lib().smoe_expert_delta(ctypes.byref(ex), msg_bf16.data_ptr(), idx.data_ptr(),
                                        w.data_ptr(), n, k, out.data_ptr(), n8.F32, ws.data_ptr(),
                                        need, n8.stream_of(torch.device(dev))), "expert_delta")
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("act", ["gelu", "swiglu"])
def test_fp8_experts_every_code(act):
    """fp8 weights holding every finite e4m3 code (subnormals, max) decode
    exactly as torch.float8_e4m3fn does (checked through the FFN output)."""
    from spider_moe_amd.quant import interleave_gate_up, interleave_gate_up_rows
    n8 = nat()
    say("fp8 experts", act)
    n, h, u, e, k = 96, 128, 128, 3, 2
    rng = np.random.default_rng(7)
    finite = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    nup = 2 * u if act == "swiglu" else u
    cu = rng.choice(finite, size=(e, nup, h)).astype(np.uint8)
    cd = rng.choice(finite, size=(e, h, u)).astype(np.uint8)
    su = (rng.random((e, nup)) * 2e-4 + 1e-5).astype(np.float32)
    sd = (rng.random((e, h)) * 2e-4 + 1e-5).astype(np.float32)
    g = torch.Generator().manual_seed(3)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    idx = torch.randint(0, e, (n, k), generator=g).to(torch.int32)
    w = torch.rand(n, k, generator=g)
    wu_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cu, su))
    wd_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cd, sd))
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx.long(), w, wu_f[:, u:], None, wd_f, None, w_gate=wu_f[:, :u])
        cu_t = interleave_gate_up(torch.from_numpy(cu[:, :u]), torch.from_numpy(cu[:, u:]))
        su_t = interleave_gate_up_rows(torch.from_numpy(su[:, :u]), torch.from_numpy(su[:, u:]))
        actc = n8.ACT_SWIGLU
    else:
        ref = _oracle_delta(msg.float(), idx.long(), w, wu_f, None, wd_f, None)
        cu_t, su_t = torch.from_numpy(cu), torch.from_numpy(su)
        actc = n8.ACT_GELU
    t = [x.contiguous().to(dev) for x in (cu_t, torch.from_numpy(cd), su_t, torch.from_numpy(sd))]
    ex = _experts_struct(n8, n8.FP8_E4M3, actc, e, h, u, t[0], t[1], s_up=t[2], s_down=t[3],
                         scale_dtype=n8.F32)
    got = _run_delta(n8, ex, msg.to(dev), idx.to(dev), w.to(dev))
    scale = ref.abs().max()
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max() <= 2e-2 * scale + 1e-6, float((got - ref).abs().max() / scale)


@pytest.mark.parametrize("act,n", [("gelu", 2304), ("swiglu", 2304), ("swiglu", 4096),
                                   ("gelu", 1100)])
def test_large_fp8_experts_ragged_groups(act, n):
    """fp8-e4m3 experts at prefill sizes (> 256 rows per expert on average,
    skewed: empty, single-row and multi-tile experts) with their weight tile
    copies: the ping-pong kernel reads the fp8 tiles, widens them to bf16 in
    registers and scales each channel in its epilogue (at n = 1100, 275 rows
    per expert, its 128-row tiles).  Against the oracle over the dequantized
    weights, and against the general fp8 kernel (no tile copy) at the same
    bound."""
    from spider_moe_amd.quant import interleave_gate_up, interleave_gate_up_rows
    n8 = nat()
    say("large fp8 experts", act, n)
    h, u, e, k = 512, 768, 8, 2
    g = torch.Generator().manual_seed(23)
    p = torch.tensor([0.45, 0.3, 0.12, 0.08, 0.05, 0.0, 0.0, 0.0])
    idx = torch.multinomial(p.expand(n, e), k, replacement=False, generator=g)
    idx[7, 1] = 5
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    nup = 2 * u if act == "swiglu" else u
    wu = torch.randn(e, nup, h, generator=g) * 0.04
    wd = torch.randn(e, h, u, generator=g) * 0.04
    cu, su = Q.fp8_quantize_per_channel(wu.numpy())
    cd, sd = Q.fp8_quantize_per_channel(wd.numpy())
    wu_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cu, su))
    wd_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cd, sd))
    bu = torch.randn(e, u, generator=g) * 0.1
    bd = torch.randn(e, h, generator=g) * 0.1
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx, w, wu_f[:, u:], bu, wd_f, bd, w_gate=wu_f[:, :u])
        cu_t = interleave_gate_up(torch.from_numpy(cu[:, :u]), torch.from_numpy(cu[:, u:]))
        su_t = interleave_gate_up_rows(torch.from_numpy(su[:, :u]), torch.from_numpy(su[:, u:]))
        actc = n8.ACT_SWIGLU
    else:
        ref = _oracle_delta(msg.float(), idx, w, wu_f, bu, wd_f, bd)
        cu_t, su_t = torch.from_numpy(cu), torch.from_numpy(su)
        actc = n8.ACT_GELU
    t = [x.contiguous().to(dev) for x in (cu_t, torch.from_numpy(cd), su_t, torch.from_numpy(sd),
                                          bu, bd)]
    ex = _experts_struct(n8, n8.FP8_E4M3, actc, e, h, u, t[0], t[1], s_up=t[2], s_down=t[3],
                         b_up=t[4], b_down=t[5], scale_dtype=n8.F32)
    plain = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    tu, td = _tiles(n8, t[0], n8.FP8_E4M3), _tiles(n8, t[1], n8.FP8_E4M3)
    ex.w_up_tiles, ex.w_down_tiles = tu.data_ptr(), td.data_ptr()
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    scale = ref.abs().max()
    assert torch.isfinite(got).all()
    for out in (got, plain):
        assert (out - ref).abs().max() <= 2e-2 * scale + 1e-6, float((out - ref).abs().max() / scale)


def _int4_qtiles_ref(packed: torch.Tensor) -> torch.Tensor:
    """The int4 tile layout on the CPU: row 64 Q + 16 t + r, bytes
    16 st + 4 fc .. +3 of the packed row -> block (g, Q, st), tile t, lane
    16 fc + r, 4 bytes each."""
    g, n, kb = packed.shape
    k = 2 * kb
    p = packed.reshape(g, n // 64, 4, 16, k // 32, 4, 4)  # g, Q, t, r, st, fc, byte
    return p.permute(0, 1, 4, 2, 5, 3, 6).contiguous().reshape(-1)


@pytest.mark.parametrize("n,kd", [(64, 32), (192, 256), (128, 2816)])
def test_pack_int4_qtiles_layout(n, kd):
    """smoe_pack_int4_qtiles rearranges the packed bytes into the int4 tile
    layout, byte for byte (checked against the layout written out on the
    CPU), and holds every byte exactly once."""
    from spider_moe_amd.quant import quantize_int4
    n8 = nat()
    say("pack int4 qtiles", n, kd)
    w = torch.randn(3, n, kd, generator=torch.Generator().manual_seed(9)) * 0.05
    q = quantize_int4(w, 32, torch.float32)
    qp = q.packed.contiguous()
    got = torch.empty_like(qp, device=dev)
    n8.check(n8.lib().smoe_pack_int4_qtiles(qp.to(dev).data_ptr(), 3, n, kd, got.data_ptr(),
                                            n8.stream_of(torch.device(dev))), "pack_int4_qtiles")
    torch.cuda.synchronize()
    want = _int4_qtiles_ref(qp)
    assert torch.equal(got.cpu().reshape(-1), want)
    assert torch.equal(torch.sort(want).values, torch.sort(qp.reshape(-1)).values)


@pytest.mark.parametrize("act,n", [("gelu", 2304), ("swiglu", 2304), ("swiglu", 1100)])
def test_large_int4_experts_ragged_groups(act, n):
    """int4 experts (group 128, fp16 scales) at prefill sizes with skewed
    routing, with their int4 tile copy: the ping-pong GEMM (256-row tiles,
    nibbles widened in registers) against the oracle over the dequantized
    weights, and against the general int4 kernel (no tiles), which
    multiplies the same bf16(q * s) values: equal to f32 summation order."""
    from spider_moe_amd.quant import interleave_gate_up, quantize_int4
    n8 = nat()
    say("large int4 experts", act, n)
    h, u, e, k, group = 512, 768, 8, 2, 128
    g = torch.Generator().manual_seed(29)
    p = torch.tensor([0.45, 0.3, 0.12, 0.08, 0.05, 0.0, 0.0, 0.0])
    idx = torch.multinomial(p.expand(n, e), k, replacement=False, generator=g)
    idx[7, 1] = 5
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    nup = 2 * u if act == "swiglu" else u
    qu = quantize_int4(torch.randn(e, nup, h, generator=g) * 0.04, group, torch.float16)
    qd = quantize_int4(torch.randn(e, h, u, generator=g) * 0.04, group, torch.float16)
    wu_f = torch.from_numpy(Q.int4_dequantize(qu.packed.numpy(), qu.scales.float().numpy(), group))
    wd_f = torch.from_numpy(Q.int4_dequantize(qd.packed.numpy(), qd.scales.float().numpy(), group))
    bu = torch.randn(e, u, generator=g) * 0.1
    bd = torch.randn(e, h, generator=g) * 0.1
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx, w, wu_f[:, u:], bu, wd_f, bd, w_gate=wu_f[:, :u])
        pu = interleave_gate_up(qu.packed[:, :u], qu.packed[:, u:])
        su = interleave_gate_up(qu.scales[:, :u], qu.scales[:, u:])
        actc = n8.ACT_SWIGLU
    else:
        ref = _oracle_delta(msg.float(), idx, w, wu_f, bu, wd_f, bd)
        pu, su = qu.packed, qu.scales
        actc = n8.ACT_GELU
    t = [x.contiguous().to(dev) for x in (pu, qd.packed, su, qd.scales, bu, bd)]
    ex = _experts_struct(n8, n8.INT4, actc, e, h, u, t[0], t[1], s_up=t[2], s_down=t[3],
                         b_up=t[4], b_down=t[5], group=group, scale_dtype=n8.F16)
    plain = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    tiles = []
    for q_ in (t[0], t[1]):
        out = torch.empty_like(q_)
        n8.check(n8.lib().smoe_pack_int4_qtiles(q_.data_ptr(), q_.shape[0], q_.shape[1],
                                                2 * q_.shape[2], out.data_ptr(),
                                                n8.stream_of(torch.device(dev))), "pack_int4_qtiles")
        tiles.append(out)
    ex.w_up_tiles, ex.w_down_tiles = tiles[0].data_ptr(), tiles[1].data_ptr()
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    scale = ref.abs().max()
    assert torch.isfinite(got).all()
    for out in (got, plain):
        assert (out - ref).abs().max() <= 2e-2 * scale + 1e-6, float((out - ref).abs().max() / scale)
    # the same bf16 weights on both kernels: only the f32 summation order differs
    assert (got - plain).abs().max() <= 2e-3 * scale, float((got - plain).abs().max() / scale)


@pytest.mark.parametrize("act,group,sdt,h", [("gelu", 32, torch.float32, 384),
                                             ("gelu", 128, torch.float16, 384),
                                             ("swiglu", 64, torch.float16, 384),
                                             ("gelu", 32, torch.float16, 448)])
def test_stream_int4_experts_ragged_passes(act, group, sdt, h):
    """int4 experts at the weight-streaming GEMM's row counts (60 rows per
    expert on average) with groups of 0, 1, 18, 96, 97 and 150 rows: one
    pass of 1, 2 and 6 live 16-row tiles, two passes with a 1-row and a
    54-row second pass; U = 640 leaves half of the last 256-channel strip
    (GELU up, 640 channels) past N_out, H = 384 half of the down GEMM's; H
    = 448 gives the up GEMM an odd number of 64-k chunks (7)."""
    from spider_moe_amd.quant import interleave_gate_up, quantize_int4
    n8 = nat()
    say("stream int4 experts", act, group, sdt, h)
    u, e, k = 640, 6, 2
    counts = [0, 1, 18, 96, 97, 150]
    flat = torch.tensor(sum(([x] * c for x, c in enumerate(counts)), []))
    n = flat.numel() // k
    idx = torch.stack([flat[:n], flat[n:]], 1)  # two different experts per token
    assert (idx[:, 0] != idx[:, 1]).all()
    g = torch.Generator().manual_seed(41)
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    nup = 2 * u if act == "swiglu" else u
    qu = quantize_int4(torch.randn(e, nup, h, generator=g) * 0.05, group, sdt)
    qd = quantize_int4(torch.randn(e, h, u, generator=g) * 0.04, group, sdt)
    wu_f = torch.from_numpy(Q.int4_dequantize(qu.packed.numpy(), qu.scales.float().numpy(), group))
    wd_f = torch.from_numpy(Q.int4_dequantize(qd.packed.numpy(), qd.scales.float().numpy(), group))
    bu = torch.randn(e, u, generator=g) * 0.1
    bd = torch.randn(e, h, generator=g) * 0.1
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx, w, wu_f[:, u:], bu, wd_f, bd, w_gate=wu_f[:, :u])
        pu = interleave_gate_up(qu.packed[:, :u], qu.packed[:, u:])
        su = interleave_gate_up(qu.scales[:, :u], qu.scales[:, u:])
        actc = n8.ACT_SWIGLU
    else:
        ref = _oracle_delta(msg.float(), idx, w, wu_f, bu, wd_f, bd)
        pu, su = qu.packed, qu.scales
        actc = n8.ACT_GELU
    t = [x.contiguous().to(dev) for x in (pu, qd.packed, su, qd.scales, bu, bd)]
    ex = _experts_struct(n8, n8.INT4, actc, e, h, u, t[0], t[1], s_up=t[2], s_down=t[3],
                         b_up=t[4], b_down=t[5], group=group,
                         scale_dtype=n8.F16 if sdt == torch.float16 else n8.F32)
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    scale = ref.abs().max()
    assert torch.isfinite(got).all()
    assert (got - ref).abs().max() <= 1e-2 * scale + 1e-6, float((got - ref).abs().max() / scale)
    one = (idx == 1).any(1)  # the token of the one-row expert
    assert one.sum() == 1 and (got[one] - ref[one]).abs().max() <= 1e-2 * scale + 1e-6


def test_stream_int4_strip_width_keeps_bits():
    """The int4 stream GEMM's strip width (192 or 256 channels) follows the
    grid: H = 2048 output channels over 64 groups fill the two workgroup
    slots per CU with 256-channel strips, over 32 groups the launcher takes
    192.  The same 32 experts and routing, once alone and once with 32
    more experts that no token chooses, must give the same bits (each output
    is summed in the same order whatever the width), and the oracle's
    values within the int4 tolerance."""
    from spider_moe_amd.quant import quantize_int4
    n8 = nat()
    say("stream int4 strip width")
    h, u, n, k, group = 2048, 256, 1536, 2, 128  # 48 / 96 rows per group: the stream kernel
    g = torch.Generator().manual_seed(43)
    first = torch.randint(0, 32, (n,), generator=g)
    idx = torch.stack([first, (first + 1 + torch.randint(0, 31, (n,), generator=g)) % 32], 1)
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    qu = quantize_int4(torch.randn(64, u, h, generator=g) * 0.05, group, torch.float16)
    qd = quantize_int4(torch.randn(64, h, u, generator=g) * 0.05, group, torch.float16)
    bu = torch.randn(64, u, generator=g) * 0.1
    bd = torch.randn(64, h, generator=g) * 0.1
    outs = []
    for e in (32, 64):
        t = [x[:e].contiguous().to(dev) for x in (qu.packed, qd.packed, qu.scales, qd.scales, bu, bd)]
        ex = _experts_struct(n8, n8.INT4, n8.ACT_GELU, e, h, u, t[0], t[1], s_up=t[2], s_down=t[3],
                             b_up=t[4], b_down=t[5], group=group, scale_dtype=n8.F16)
        outs.append(_run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev)))
    assert torch.equal(outs[0], outs[1])
    wu_f = torch.from_numpy(Q.int4_dequantize(qu.packed[:32].numpy(), qu.scales[:32].float().numpy(), group))
    wd_f = torch.from_numpy(Q.int4_dequantize(qd.packed[:32].numpy(), qd.scales[:32].float().numpy(), group))
    ref = _oracle_delta(msg.float(), idx, w, wu_f, bu[:32], wd_f, bd[:32])
    scale = ref.abs().max()
    assert (outs[0] - ref).abs().max() <= 1e-2 * scale + 1e-6, float((outs[0] - ref).abs().max() / scale)


@pytest.mark.parametrize("group,sdt", [(32, torch.float32), (128, torch.float16)])
def test_int4_experts_match_oracle(group, sdt):
    from spider_moe_amd.quant import quantize_int4
    n8 = nat()
    say("int4 experts", group, sdt)
    msg, idx, w, wu, bu, wd, bd = _delta_case(200, 256, 384, 5, 2, 11, scale=0.05)
    qu, qd = quantize_int4(wu, group, sdt), quantize_int4(wd, group, sdt)
    wu_f = torch.from_numpy(Q.int4_dequantize(qu.packed.numpy(), qu.scales.float().numpy(), group))
    wd_f = torch.from_numpy(Q.int4_dequantize(qd.packed.numpy(), qd.scales.float().numpy(), group))
    msg = msg.to(torch.bfloat16)
    ref = _oracle_delta(msg.float(), idx, w, wu_f, bu, wd_f, bd)
    t = [x.contiguous().to(dev) for x in (qu.packed, qd.packed, qu.scales, qd.scales, bu, bd)]
    ex = _experts_struct(n8, n8.INT4, n8.ACT_GELU, 5, 256, 384, t[0], t[1], s_up=t[2], s_down=t[3],
                         b_up=t[4], b_down=t[5], group=group,
                         scale_dtype=n8.F16 if sdt == torch.float16 else n8.F32)
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    torch.testing.assert_close(got, ref, rtol=1e-2, atol=1e-2)
    # the quantization error envelope the reference accepts (dequant vs fp weights)
    ref_fp = _oracle_delta(msg.float(), idx, w, wu, bu, wd, bd)
    env = (ref - ref_fp).abs().max()
    assert (got - ref).abs().max() < max(float(env), 1e-3)


@pytest.mark.parametrize("shape", [(24, 384, 640, 8), (60, 384, 640, 8), (40, 768, 1664, 4),
                                   (20, 256, 640, 8), (180, 384, 640, 6), (180, 64, 128, 6)])
@pytest.mark.parametrize("fmt,act", [("bf16", "gelu"), ("bf16", "swiglu"), ("fp8", "gelu"),
                                     ("fp8", "swiglu"), ("int4-g32-f32", "gelu"),
                                     ("int4-g128-f16", "gelu")])
def test_decode_experts_match_oracle(fmt, act, shape):
    """Decode shapes (a few rows per expert) take the weight-streaming GEMM,
    K split over 1, 2 or 4 waves with ragged parts: up K = 256 (4 steps of
    64: no split), 384 (6) and 768 (12), down K = 640 (10) and 1664 (26:
    parts of 6 and 7 steps, so the ring's main loop runs); 16-row tiles (6
    rows per expert on average) and 32-row tiles (15 and 20); an expert with
    more rows than one tile holds, an empty expert, a one-row expert.  At
    (180, 384, 640, 6) the experts hold 60 rows on average, the shape of the
    medium-size stream GEMMs (a 256-channel strip over all of an expert's
    rows), and expert 0's 180 rows take several passes; (180, 64, 128, 6)
    gives the up GEMM a single 64-k chunk."""
    from spider_moe_amd.quant import interleave_gate_up, interleave_gate_up_rows, quantize_int4
    n8 = nat()
    say("decode experts", fmt, act, shape)
    n, h, u, e = shape
    if "g128" in fmt and h % 128:
        pytest.skip("int4 group 128 needs H % 128 == 0")
    k = 2
    g = torch.Generator().manual_seed(31)
    idx = torch.zeros(n, k, dtype=torch.long)
    idx[:, 1] = 1 + torch.randperm(n, generator=g) % (e - 3)  # experts 1 .. e-3
    idx[5, 1] = e - 1            # expert e-1: one row;  expert e-2: none
    # expert 0: every token (more rows than one tile)
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    nup = 2 * u if act == "swiglu" else u
    # weights scaled by 1/sqrt(K) (0.05 at K = 384 / 640) so the outputs, and
    # with them what the absolute tolerance allows, keep one size across shapes
    wu = torch.randn(e, nup, h, generator=g) * (0.05 * (384 / h) ** 0.5)
    wd = torch.randn(e, h, u, generator=g) * (0.05 * (640 / u) ** 0.5)
    bu = torch.randn(e, u, generator=g) * 0.1
    bd = torch.randn(e, h, generator=g) * 0.1
    kw = {}
    if fmt == "bf16":
        wu, wd = wu.to(torch.bfloat16), wd.to(torch.bfloat16)
        wu_f, wd_f = wu.float(), wd.float()
        code, dev_up, dev_dn = n8.BF16, wu, wd
    elif fmt == "fp8":
        cu, su = Q.fp8_quantize_per_channel(wu.numpy())
        cd, sd = Q.fp8_quantize_per_channel(wd.numpy())
        wu_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cu, su))
        wd_f = torch.from_numpy(Q.fp8_dequantize_per_channel(cd, sd))
        code, dev_up, dev_dn = n8.FP8_E4M3, torch.from_numpy(cu), torch.from_numpy(cd)
        su_t = torch.from_numpy(su).float()
        kw = dict(s_up=su_t, s_down=torch.from_numpy(sd).float(), scale_dtype=n8.F32)
    else:
        group = 32 if "g32" in fmt else 128
        sdt = torch.float32 if "f32" in fmt else torch.float16
        qu, qd = quantize_int4(wu, group, sdt), quantize_int4(wd, group, sdt)
        wu_f = torch.from_numpy(Q.int4_dequantize(qu.packed.numpy(), qu.scales.float().numpy(), group))
        wd_f = torch.from_numpy(Q.int4_dequantize(qd.packed.numpy(), qd.scales.float().numpy(), group))
        # the device widens q * s to bf16 once (fp32 product, RNE)
        wu_f, wd_f = B.round_bf16(wu_f), B.round_bf16(wd_f)
        code, dev_up, dev_dn = n8.INT4, qu.packed, qd.packed
        kw = dict(s_up=qu.scales, s_down=qd.scales, group=group,
                  scale_dtype=n8.F16 if sdt == torch.float16 else n8.F32)
    # the device keeps the FFN hidden activation in bf16: model that rounding
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx, w, wu_f[:, u:], bu, wd_f, bd, w_gate=wu_f[:, :u],
                            hidden_bf16=True)
        dev_up = interleave_gate_up(dev_up[:, :u], dev_up[:, u:])
        if "s_up" in kw:
            kw["s_up"] = interleave_gate_up_rows(kw["s_up"][:, :u], kw["s_up"][:, u:])
    else:
        ref = _oracle_delta(msg.float(), idx, w, wu_f, bu, wd_f, bd, hidden_bf16=True)
    kw = {a: (v.contiguous().to(dev) if torch.is_tensor(v) else v) for a, v in kw.items()}
    up_d, dn_d = dev_up.contiguous().to(dev), dev_dn.contiguous().to(dev)
    bu_d, bd_d = bu.to(dev), bd.to(dev)
    ex = _experts_struct(n8, code, n8.ACT_SWIGLU if act == "swiglu" else n8.ACT_GELU, e, h, u,
                         up_d, dn_d, b_up=bu_d, b_down=bd_d, **kw)
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    torch.testing.assert_close(got, ref, rtol=1e-2, atol=1e-2)
    if fmt in ("bf16", "fp8"):  # the weight tile layout: the same fragments, so the same bits
        tu, td = _tiles(n8, up_d, code), _tiles(n8, dn_d, code)
        ex.w_up_tiles, ex.w_down_tiles = tu.data_ptr(), td.data_ptr()
        got_t = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
        assert torch.equal(got_t, got)


def test_invalid_arguments_are_rejected():
    n8 = nat()
    say("invalid args")
    ex = n8.SmoeExperts()
    ex.w_up = ex.w_down = ex.s_up = ex.s_down = 256  # never dereferenced by the size query
    ex.format, ex.E, ex.H, ex.U = n8.FP8_E4M3, 4, 100, 64  # fp8: H not a multiple of 32
    assert n8.lib().smoe_expert_delta_workspace_bytes(ctypes.byref(ex), 10, 2) == 0
    ex.format, ex.act = n8.BF16, n8.ACT_SWIGLU  # SwiGLU pairs need the MFMA grid too
    assert n8.lib().smoe_expert_delta_workspace_bytes(ctypes.byref(ex), 10, 2) == 0
    ex.act = n8.ACT_GELU  # bf16 GELU takes any H (the SIMT kernel)
    assert n8.lib().smoe_expert_delta_workspace_bytes(ctypes.byref(ex), 10, 2) > 0
    ex.E = 257  # E > 256
    assert n8.lib().smoe_expert_delta_workspace_bytes(ctypes.byref(ex), 10, 2) == 0
    rc = n8.lib().smoe_router_topk(None, n8.BF16, 4, 64, None, None, 4, 5, None, None, None, None,
                                   0, None)
    assert rc == 1


@pytest.mark.parametrize("act,u,n", [("gelu", 768, 2304), ("swiglu", 768, 2304), ("gelu", 640, 2304),
                                     ("gelu", 768, 4096), ("swiglu", 768, 4096),
                                     ("swiglu", 704, 2304), ("gelu", 768, 1536), ("swiglu", 768, 1536),
                                     ("gelu", 1024, 1100), ("gelu", 768, 1200), ("swiglu", 768, 1200)])
def test_large_bf16_experts_ragged_groups(act, u, n):
    """Shapes that take the large-tile LDS-DMA paths (> 128 rows per expert
    on average) with skewed routing: empty experts, single-row experts and
    experts spanning several tiles.  With n = 2304 / 4096 (576 / 1024 rows
    per expert on average) up N_out 768 / 1536 and down N_out 512 (multiples
    of 256) take the 8-wave ping-pong kernel with 256- / 320-row tiles, up
    N_out 640 / 1408 (odd multiples of 128) the 256 x 128 ring kernel.  With
    n = 1536 / 1100 (384 / 275 rows per expert; groups of 0, 1, ~100-400 and
    ~1000 rows) the ping-pong kernel takes 128-row tiles, with n = 1200 (300
    rows per expert) its 320-row tiles."""
    from spider_moe_amd.quant import interleave_gate_up
    n8 = nat()
    say("large bf16 experts", act, u, n)
    h, e, k = 512, 8, 2
    g = torch.Generator().manual_seed(21)
    # skew: experts 0,1 take most tokens, 5 gets one token, 6 and 7 none
    p = torch.tensor([0.45, 0.3, 0.12, 0.08, 0.05, 0.0, 0.0, 0.0])
    idx = torch.multinomial(p.expand(n, e), k, replacement=False, generator=g)
    idx[7, 1] = 5
    w = torch.rand(n, k, generator=g)
    msg = torch.randn(n, h, generator=g).to(torch.bfloat16)
    nup = 2 * u if act == "swiglu" else u
    wu = (torch.randn(e, nup, h, generator=g) * 0.04).to(torch.bfloat16)
    wd = (torch.randn(e, h, u, generator=g) * 0.04).to(torch.bfloat16)
    bu = torch.randn(e, u, generator=g) * 0.1 if act == "gelu" else None
    bd = torch.randn(e, h, generator=g) * 0.1 if act == "gelu" else None
    if act == "swiglu":
        ref = _oracle_delta(msg.float(), idx, w, wu.float()[:, u:], None, wd.float(), None,
                            w_gate=wu.float()[:, :u])
        wu_dev = interleave_gate_up(wu[:, :u], wu[:, u:]).to(dev)
    else:
        ref = _oracle_delta(msg.float(), idx, w, wu.float(), bu, wd.float(), bd)
        wu_dev = wu.to(dev)
    wd_dev = wd.contiguous().to(dev)
    bu_d = bu.to(dev) if bu is not None else None
    bd_d = bd.to(dev) if bd is not None else None
    ex = _experts_struct(n8, n8.BF16, n8.ACT_SWIGLU if act == "swiglu" else n8.ACT_GELU, e, h, u,
                         wu_dev, wd_dev, b_up=bu_d, b_down=bd_d)
    got = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    torch.testing.assert_close(got, ref, rtol=1e-2, atol=1e-2)
    # the ping-pong kernel with its W operand read from the weight tile copy
    # (lane-ordered 1 KB fragment blocks): the same fragments, the same bits
    tu, td = _tiles(n8, wu_dev), _tiles(n8, wd_dev)
    ex.w_up_tiles, ex.w_down_tiles = tu.data_ptr(), td.data_ptr()
    got_t = _run_delta(n8, ex, msg.to(dev), idx.to(torch.int32).to(dev), w.to(dev))
    assert torch.equal(got_t, got)
