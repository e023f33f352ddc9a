"""GPU parity of the reference's device ABI (spider_cuda_* through
HipKernels / NativeLoop) against oracle/native.py, and of the Forge
surfaces (ForgeSelect, ForgeGEMM, dispatch_expert_ffn with an expert_fn)
against oracle/forge.py.

Tolerances: the device ABI follows the scalar library's operation order;
what remains are libm differences (expf in the router, tanhf in the GELU)
and the router's sum order (a wave reduction against index order), so
router weights compare at rtol 1e-5, expert outputs at rtol 1e-4 and the
epilogue (a two-pass double variance against Welford) at 1e-5; the graph
pass, indices, masks and the dispatch combine (fp32 and bf16) are exact."""
import numpy as np
import pytest
import torch

from oracle import forge as OF
from oracle import native as ON

pytestmark = pytest.mark.gpu

dev = "cuda"


def say(*a):
    print("[case]", *a, flush=True)


def _kern():
    from spider_moe_amd.native_compat import HipKernels
    return HipKernels(dev)


def _rng(seed):
    return np.random.default_rng(seed)


# ----------------------------------------------------- device ABI ----
@pytest.mark.parametrize("b,e,k", [(2, 4, 2), (300, 16, 2), (77, 64, 8), (5, 33, 3), (50, 100, 4),
                                   (9, 256, 8)])
def test_spider_cuda_router(b, e, k):
    say("spider_cuda_router", b, e, k)
    kern = _kern()
    r = _rng(e + k)
    logits = r.standard_normal((b, e)).astype(np.float32)
    bias = (0.1 * r.standard_normal((3, e))).astype(np.float32)
    for loop in (0, 2):
        w, i = kern.router(logits, bias, k, loop)
        wo, io = ON.router(logits, bias[loop], k)
        assert np.array_equal(i, io)
        assert np.allclose(w, wo, rtol=1e-5, atol=1e-7)
    if b == 2:  # kernels/tests/test_kernels.cpp:7-18
        w, i = kern.router(np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float32),
                           np.zeros((1, 4), np.float32), 2)
        assert i.tolist() == [[3, 2], [0, 1]]
        assert np.allclose(w.sum(-1), 1.0, atol=1e-6)


def test_spider_cuda_argument_errors():
    kern = _kern()
    with pytest.raises(RuntimeError, match="spider_cuda_router_f32 failed"):
        kern.router(np.zeros((2, 4), np.float32), np.zeros((1, 4), np.float32), 5)
    with pytest.raises(RuntimeError, match="spider_cuda_router_f32 failed"):
        kern.router(np.zeros((2, 300), np.float32), np.zeros((1, 300), np.float32), 2)


def _csr(e, r, fanout=3):
    rp = [0]
    ci = []
    for s in range(e):
        n = int(r.integers(0, fanout + 1))
        ci += [int(x) for x in r.integers(0, e, n)]
        rp.append(len(ci))
    return np.array(rp, np.int32), np.array(ci, np.int32)


@pytest.mark.parametrize("b,h,e,k", [(5, 16, 6, 2), (200, 256, 16, 2), (33, 1000, 32, 4)])
def test_spider_cuda_graph_v1(b, h, e, k):
    say("spider_cuda_graph", b, h, e, k)
    kern = _kern()
    r = _rng(h)
    x = r.standard_normal((b, h)).astype(np.float32)
    rp, ci = _csr(e, r)
    nnz = len(ci)
    ew = r.random(2 * nnz).astype(np.float32)
    asg = r.integers(0, e, (b, k)).astype(np.int32)
    asg[0, -1] = -1  # an empty slot is skipped
    rw = r.random((b, k)).astype(np.float32)
    for loop in (0, 1):
        got = kern.graph(x, rp, ci, ew, asg, rw, e, loop)
        want = ON.graph_v1(x, rp, ew, asg, rw, nnz=nnz, loop_idx=loop)
        assert np.array_equal(got, want)


@pytest.mark.parametrize("workspace", [False, True])
@pytest.mark.parametrize("b,h,u,e,k", [(5, 32, 24, 4, 2), (64, 256, 512, 8, 2), (9, 200, 72, 5, 3)])
def test_spider_cuda_expert_ffn(workspace, b, h, u, e, k):
    say("spider_cuda_expert", workspace, b, h, u, e, k)
    kern = _kern()
    r = _rng(h + u)
    x = r.standard_normal((b, h)).astype(np.float32)
    wu = (r.standard_normal((e, h, u)) / np.sqrt(h)).astype(np.float32)
    wd = (r.standard_normal((e, u, h)) / np.sqrt(u)).astype(np.float32)
    asg = r.integers(0, e, (b, k)).astype(np.int32)
    asg[1, 0] = -1
    rw = r.random((b, k)).astype(np.float32)
    got = kern.expert_ffn(x, asg, rw, wu, wd, e, workspace=workspace)
    want = ON.experts(x, asg, rw, wu, wd)
    assert np.allclose(got, want, rtol=1e-4, atol=1e-5)
    assert np.abs(want).max() > 0.1


@pytest.mark.parametrize("b,h", [(8, 48), (300, 1024), (3, 4000)])
def test_spider_cuda_epilogue_and_exit(b, h):
    say("spider_cuda_epilogue", b, h)
    kern = _kern()
    r = _rng(h)
    hh, d, x0 = (r.standard_normal((b, h)).astype(np.float32) for _ in range(3))
    g = (1 + 0.1 * r.standard_normal(h)).astype(np.float32)
    lb = (0.1 * r.standard_normal(h)).astype(np.float32)
    got = kern.epilogue(hh, d, x0, g, lb, 0.5, 0.1, 1e-5)
    want = ON.epilogue(hh, d, x0, 0.5, 0.1, g, lb, 1e-5)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    proj = (r.standard_normal(h) / np.sqrt(h)).astype(np.float32)
    for thr in (0.3, 0.5, 0.8):
        mask = kern.early_exit(want, proj, thr)
        mo, conf = ON.exit_mask(want, proj, thr)
        far = np.abs(conf - thr) > 1e-5
        assert np.array_equal(mask[far], mo[far])


@pytest.mark.parametrize("graph", [False, True])
@pytest.mark.parametrize("b,h,u,e,k", [(7, 32, 24, 8, 2), (128, 512, 256, 16, 2)])
def test_spider_cuda_moe_loop_step(graph, b, h, u, e, k):
    say("spider_cuda_loop_step", graph, b, h, u, e, k)
    kern = _kern()
    r = _rng(b + h)
    hh, x0 = (r.standard_normal((b, h)).astype(np.float32) for _ in range(2))
    rw = (r.standard_normal((h, e)) / np.sqrt(h)).astype(np.float32)
    bias = (0.1 * r.standard_normal((1, e))).astype(np.float32)
    wu = (r.standard_normal((e, h, u)) / np.sqrt(h)).astype(np.float32)
    wd = (r.standard_normal((e, u, h)) / np.sqrt(u)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(h)).astype(np.float32)
    lb = (0.1 * r.standard_normal(h)).astype(np.float32)
    proj = (r.standard_normal(h) / np.sqrt(h)).astype(np.float32)
    csr = None
    if graph:
        rp, ci = _csr(e, r)
        csr = (rp, ci, r.random(len(ci)).astype(np.float32))
    hn, mask, asg, route = kern.moe_loop_step(hh, x0, 0, router_w=rw, loop_bias=bias, W_up=wu,
                                              W_down=wd, ln_weight=g, ln_bias=lb, top_k=k,
                                              alpha=0.5, beta=0.1, csr=csr, exit_proj=proj,
                                              exit_threshold=0.5)
    wn, wm, wa, wr, _ = ON.loop_step(hh, x0, k, rw, bias[0], wu, wd, g, lb, 0.5, 0.1, 1e-5,
                                     csr=csr, exit_proj=proj, threshold=0.5)
    assert np.array_equal(asg, wa)
    assert np.allclose(route, wr, rtol=1e-5, atol=1e-7)
    assert np.allclose(hn, wn, rtol=1e-4, atol=1e-4)
    _, conf = ON.exit_mask(wn, proj, 0.5)
    far = np.abs(conf - 0.5) > 1e-4
    assert np.array_equal(mask[far], wm[far])


def test_native_loop_runs_a_spiderw_bundle(tmp_path):
    """NativeLoop over a bundle written to disk: every loop equals the
    oracle's loop step (static CSR graph with per-loop edge weights, exit
    head present but early exit off)."""
    from spider_moe_amd.native_compat import NativeLoop
    from spider_moe_amd.spiderw import SpiderWMeta, write_spiderw
    say("native_loop bundle")
    r = _rng(11)
    h, e, k, u, loops, b = 64, 8, 2, 96, 3, 20
    rp, ci = _csr(e, r)
    t = {"router": (r.standard_normal((h, e)) / np.sqrt(h)).astype(np.float32),
         "loop_bias": (0.1 * r.standard_normal((loops, e))).astype(np.float32),
         "expert_up": (r.standard_normal((e, h, u)) / np.sqrt(h)).astype(np.float32),
         "expert_down": (r.standard_normal((e, u, h)) / np.sqrt(u)).astype(np.float32),
         "moe_norm": np.stack([1 + 0.1 * r.standard_normal(h),
                               0.1 * r.standard_normal(h)]).astype(np.float32),
         "exit_head": (r.standard_normal(h) / np.sqrt(h)).astype(np.float32),
         "csr_row_ptr": rp, "csr_col_idx": ci,
         "csr_edge_w": r.random(loops * len(ci)).astype(np.float32)}
    meta = SpiderWMeta(flags=2, hidden_size=h, num_experts=e, top_k=k, num_loops=loops,
                       expert_ffn_size=u)
    p = tmp_path / "block.spiderw"
    write_spiderw(p, meta, t)
    nl = NativeLoop(str(p))
    x = r.standard_normal((b, h)).astype(np.float32)
    got = nl.run_loops(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = x
    nnz = len(ci)
    for loop in range(loops):
        ew = t["csr_edge_w"][loop * nnz:(loop + 1) * nnz]
        want = ON.loop_step(want, x, k, t["router"], t["loop_bias"][loop], t["expert_up"],
                            t["expert_down"], t["moe_norm"][0], t["moe_norm"][1], 0.5, 0.1, 1e-5,
                            csr=(rp, ci, ew))[0]
    assert np.allclose(got, want, rtol=1e-3, atol=1e-3)


# ---------------------------------------------------------- forge ----
@pytest.mark.parametrize("n,e,k", [(1, 4, 2), (500, 16, 2), (1000, 64, 6), (37, 40, 40),
                                   (300, 200, 5), (50, 256, 64), (70, 65, 1)])
def test_forge_select_route(n, e, k):
    from spider_moe_amd.forge import ForgeConfig, ForgeSelect
    say("forge_select", n, e, k)
    g = torch.Generator().manual_seed(n + e)
    logits = torch.randn(2, n, e, generator=g)
    sel = ForgeSelect(ForgeConfig(select_top_k=k))
    w, i = sel.route(logits.to(dev))
    wo, io = OF.select_route(logits, k)
    assert w.shape == (2, n, k) and i.dtype == torch.int64
    assert torch.equal(i.cpu(), io)
    assert torch.allclose(w.cpu(), wo, rtol=1e-5, atol=1e-7)
    # bf16 logits: weights come back in bf16
    wb, ib = sel.route(logits.to(dev, torch.bfloat16), top_k=1)
    assert wb.dtype == torch.bfloat16 and torch.all(wb == 1)


def test_select_router_mode_matches_block_router():
    """smoe_select_topk mode 0 is the block's router selection
    (model.py:255-258): top-k of the fp32 softmax, renormalised."""
    from spider_moe_amd import _native as nat
    from spider_moe_amd.forge import select_topk
    say("select router mode")
    g = torch.Generator().manual_seed(5)
    logits = torch.randn(700, 32, generator=g)
    w, i = select_topk(logits.to(dev), 4, nat.SMOE_SELECT_ROUTER)
    p = logits.softmax(-1)
    wo, io = p.topk(4, dim=-1)
    wo = wo / wo.sum(-1, keepdim=True).clamp_min(1e-9)
    assert torch.equal(i.cpu(), io)
    assert torch.allclose(w.cpu(), wo, rtol=1e-5, atol=1e-7)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,kd,no", [(3, 64, 40), (300, 256, 512), (1024, 512, 1000)])
def test_forge_gemm_linear(dtype, n, kd, no):
    from spider_moe_amd.forge import ForgeGEMM
    say("forge_linear", dtype, n, kd, no)
    g = torch.Generator().manual_seed(n + kd)
    x = torch.randn(n, kd, generator=g).to(dtype)
    w = (torch.randn(no, kd, generator=g) / kd ** 0.5).to(dtype)
    b = torch.randn(no, generator=g).to(dtype)
    got = ForgeGEMM().linear(x.to(dev), w.to(dev), b.to(dev)).cpu()
    want = OF.linear(x, w, b)
    assert got.dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert torch.allclose(got.float(), want.float(), rtol=tol, atol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,kd,no", [(5, 64, 128), (600, 512, 256)])
def test_forge_gemm_fp8_linear(dtype, n, kd, no):
    """Per-tensor fp8 weights (quantize_fp8): the codes and scale are the
    oracle's exactly; the product within the bf16 rounding of the
    activations (the reference rounds them to fp16)."""
    from spider_moe_amd.forge import ForgeGEMM
    from spider_moe_amd.quant import quantize_fp8_per_tensor
    say("forge_fp8_linear", dtype, n, kd, no)
    g = torch.Generator().manual_seed(n)
    x = torch.randn(n, kd, generator=g).to(dtype)
    w = (torch.randn(no, kd, generator=g) / kd ** 0.5)
    b = torch.randn(no, generator=g)
    codes, scale = quantize_fp8_per_tensor(w.to(dev))
    oc, osc = OF.fp8_quantize_per_tensor(w)
    assert torch.equal(codes.view(torch.uint8).cpu(), oc.view(torch.uint8))
    assert float(scale) == float(osc)  # IEEE divisions on the device, as on the CPU
    gemm = ForgeGEMM()
    got = gemm.linear_fp8(x.to(dev), w.to(dev), b.to(dev)).cpu().float()
    want = OF.fp8_linear(x, w, b).float()
    ref = (x.float() @ w.t() + b)
    err = (got - want).abs().max() / want.abs().max()
    assert err < 1.5e-2, err
    # the fp8 result stays near the unquantized product (a sanity bound)
    assert (got - ref).abs().max() / ref.abs().max() < 0.1


@pytest.mark.parametrize("per_row", [False, True])
def test_quantize_fp8_weights_match_cpu_bits(per_row):
    """Weights quantized on the device (per tensor for Forge, per output
    channel for the block's fp8 experts) give the CPU formula's scales and
    codes bit for bit, over shapes whose amax divides to scales off a
    power of two; torch's own GPU division does not (it multiplies by a
    reciprocal), which is why the HIP quantizer does it."""
    from spider_moe_amd.quant import quantize_fp8_per_channel, quantize_fp8_per_tensor
    from oracle import quant as OQ  # noqa: F401
    say("quantize weights", "per_row" if per_row else "per_tensor")
    for (r, c) in ((256, 512), (300, 1000), (1024, 2048), (7, 37)):
        g = torch.Generator().manual_seed(r + c)
        w = torch.randn(2, r, c, generator=g) / c ** 0.5
        if per_row:
            codes, scale = quantize_fp8_per_channel(w.to(dev))
            ws = (w.abs().amax(dim=-1) / 448.0).clamp_min(1e-12)
            wc = (w / ws.unsqueeze(-1)).to(torch.float8_e4m3fn)
        else:
            codes, scale = quantize_fp8_per_tensor(w.to(dev))
            wc, ws = OF.fp8_quantize_per_tensor(w)
        assert torch.equal(scale.cpu(), ws), (r, c)
        assert torch.equal(codes.view(torch.uint8).cpu(), wc.view(torch.uint8)), (r, c)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_quantize_fp8_input_matches_torch_cast(dtype):
    """smoe_quantize_fp8_tensor against quantize_fp8 (quant.py:30-56) on the
    CPU: the same scale and the same e4m3 codes bit for bit, over random
    values, exact midpoints between neighbouring codes (round to nearest
    even) in the normal and subnormal ranges, and zeros; the K padding
    holds code 0."""
    from spider_moe_amd.forge import quantize_fp8_input
    say("quantize_fp8_input", dtype)
    g = torch.Generator().manual_seed(21)
    x = torch.randn(37, 300, generator=g) * 3.0
    x[0, 0] = 448.0                      # amax: scale 1 exactly
    x[0, 1:] = 0.0
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    grid = grid[torch.isfinite(grid)].unique()            # the 253 finite values, sorted
    mids = (grid[1:] + grid[:-1]) / 2                     # exact ties, sign mixed
    mids = mids * torch.where(torch.arange(mids.numel()) % 2 == 0, 1.0, -1.0)
    x[1:1 + (mids.numel() + 299) // 300].view(-1)[:mids.numel()] = mids
    x = x.to(dtype)
    codes, scale = quantize_fp8_input(x.to(dev), 512)
    oc, osc = OF.fp8_quantize_per_tensor(x)
    assert float(scale) == float(osc)
    c = codes.cpu()
    assert torch.equal(c[:, :300], oc.view(torch.uint8)), int((c[:, :300] != oc.view(torch.uint8)).sum())
    assert int(c[:, 300:].abs().sum()) == 0
    # a scale off a power of two: the divisions themselves are compared
    y = (torch.randn(64, 300, generator=g) * 1.7).to(dtype)
    codes, scale = quantize_fp8_input(y.to(dev), 304)
    oc, osc = OF.fp8_quantize_per_tensor(y)
    assert float(scale) == float(osc)
    assert torch.equal(codes.cpu()[:, :300], oc.view(torch.uint8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,kd,no", [(5, 64, 128), (600, 512, 256), (1000, 1000, 300),
                                     (257, 2048, 1024)])
def test_forge_fp8_linear_quantize_input(dtype, n, kd, no):
    """fp8_linear(quantize_input=True) (forge/gemm/fp8.py:49-52): e4m3 x
    e4m3 on the f8f6f4 MFMA against the oracle, which dequantizes both
    operands (fp16 compute for bf16 inputs, fp32 for fp32 inputs): fp32 to
    1e-4 of the largest output, bf16 within the fp16 / bf16 roundings; K, N and
    N_out off the kernel's 256 / 128 grid."""
    from spider_moe_amd.forge import ForgeGEMM, fp8_linear, get_last_fp8_gemm_backend
    say("forge_fp8_linear quantize_input", dtype, n, kd, no)
    g = torch.Generator().manual_seed(n + kd + no)
    x = torch.randn(n, kd, generator=g).to(dtype)
    w = (torch.randn(no, kd, generator=g) / kd ** 0.5)
    b = torch.randn(no, generator=g)
    got = ForgeGEMM().linear_fp8(x.to(dev), w.to(dev), b.to(dev), quantize_input=True)
    assert got.dtype == dtype and got.shape == (n, no)
    got = got.cpu().float()
    want = OF.fp8_linear(x, w, b, quantize_input=True).float()
    err = (got - want).abs().max() / want.abs().max()
    # f32: the oracle rounds x_deq, w_deq and each product; the kernel sums
    # the exact code products and scales once
    assert err < (1e-4 if dtype == torch.float32 else 1.5e-2), err
    got2 = fp8_linear(x.to(dev), w.to(dev), b.to(dev), quantize_input=True).cpu().float()
    assert torch.equal(got2, got)
    assert get_last_fp8_gemm_backend()[0] == "hip_fp8xfp8_mfma_f8f6f4"


def test_forge_fp8_linear_quantize_input_exact_on_the_grid():
    """Inputs and weights already on the e4m3 grid of scale 1 (amax 448):
    integer codes of magnitude <= 64 (plus one 448 each), so every product
    and every partial sum is an integer below 2^24, exact in f32 in any
    order.  The f8f6f4 MFMA multiplies the codes exactly but sums each
    128-product block below f32 precision: measured within 2^-14 of the
    block's largest product (the row and column holding 448 * 448 = 200704
    are off by up to ~10); every other entry, whose products stay at or
    below 64 * 64, is exact.  A wrong k pairing or a dropped block misses
    by thousands."""
    from spider_moe_amd.forge import fp8_linear
    say("fp8 x fp8 exact")
    grid = torch.arange(256, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    grid = grid[torch.isfinite(grid) & (grid == grid.round()) & (grid.abs() <= 64)]
    g = torch.Generator().manual_seed(5)
    x = grid[torch.randint(0, grid.numel(), (70, 256), generator=g)]
    w = grid[torch.randint(0, grid.numel(), (130, 256), generator=g)]
    x[0, 0] = 448.0
    w[0, 0] = 448.0
    got = fp8_linear(x.to(dev), w.to(dev), quantize_input=True).cpu()
    want = (x.double() @ w.double().t()).float()
    assert torch.equal(got[1:, 1:], want[1:, 1:])
    big = (x.double().abs() @ w.double().abs().t()).max(dim=-1).values  # bound per row
    err = (got - want).abs().double()
    assert bool((err[0] <= 448.0 * 448.0 * 2.0 ** -13).all()), float(err[0].max())
    assert bool((err[:, 0] <= 448.0 * 448.0 * 2.0 ** -13).all()), float(err[:, 0].max())
    assert float(big.min()) > 0


def test_forge_fp8_expert_ffn_quantize_input():
    """fp8_expert_ffn(quantize_input=True) (fp8.py:65-76): the up projection
    e4m3 x e4m3 with GELU, the down projection on fp8 weights; fp32 inputs
    (the reference's fp32 compute) and bf16 inputs."""
    from spider_moe_amd.forge import fp8_expert_ffn
    for dtype in (torch.float32, torch.bfloat16):
        say("fp8_expert_ffn quantize_input", dtype)
        g = torch.Generator().manual_seed(17)
        h, u, n = 256, 512, 200
        x = torch.randn(n, h, generator=g).to(dtype)
        wu = (torch.randn(u, h, generator=g) / h ** 0.5).to(dtype)
        bu = (torch.randn(u, generator=g) * 0.1).to(dtype)
        wd = (torch.randn(h, u, generator=g) / u ** 0.5).to(dtype)
        bd = (torch.randn(h, generator=g) * 0.1).to(dtype)
        got = fp8_expert_ffn(x.to(dev), wu.to(dev), bu.to(dev), wd.to(dev), bd.to(dev),
                             quantize_input=True)
        assert got.dtype == dtype
        got = got.cpu().float()
        want = OF.fp8_expert_ffn(x, wu, bu, wd, bd, quantize_input=True).float()
        err = (got - want).abs().max() / want.abs().max()
        assert err < (1e-4 if dtype == torch.float32 else 3e-2), (dtype, err)


def test_forge_fp8_linear_f32_inputs_keep_f32():
    """f32 inputs on the fp8 weight path multiply in f32 (the reference's
    compute dtype for f32, fp8.py:41-54): the dequantized codes times x in
    f32, not x rounded to bf16."""
    from spider_moe_amd.forge import ForgeGEMM
    say("fp8 weights, f32 inputs")
    g = torch.Generator().manual_seed(8)
    x = torch.randn(300, 256, generator=g)
    w = torch.randn(200, 256, generator=g) / 16
    got = ForgeGEMM().linear_fp8(x.to(dev), w.to(dev)).cpu()
    want = OF.fp8_linear(x, w)
    assert got.dtype == torch.float32
    assert torch.allclose(got, want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("fp8", [False, True])
def test_forge_gemm_expert_ffn(fp8):
    from spider_moe_amd.forge import ForgeConfig, ForgeGEMM
    say("forge_expert_ffn", fp8)
    g = torch.Generator().manual_seed(9)
    h, u, n = 256, 512, 200
    bf = torch.bfloat16
    x = torch.randn(n, h, generator=g).to(bf)
    wu = (torch.randn(u, h, generator=g) / h ** 0.5).to(bf)
    bu = (torch.randn(u, generator=g) * 0.1).to(bf)
    wd = (torch.randn(h, u, generator=g) / u ** 0.5).to(bf)
    bd = (torch.randn(h, generator=g) * 0.1).to(bf)
    got = ForgeGEMM(ForgeConfig(gemm_fp8=fp8)).expert_ffn(
        x.to(dev), wu.to(dev), bu.to(dev), wd.to(dev), bd.to(dev))
    assert got.dtype == bf
    got = got.cpu().float()
    want = OF.expert_ffn(x, wu, bu, wd, bd, fp8).float()
    err = (got - want).abs().max() / want.abs().max()
    assert err < (3e-2 if fp8 else 2e-2), err


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,h,e,k", [(10, 8, 5, 3), (513, 256, 16, 4), (64, 1000, 8, 2)])
def test_dispatch_expert_fn_combine_is_exact(dtype, n, h, e, k):
    """dispatch_expert_ffn with an expert_fn: the callback sees each
    expert's packed rows and the weighted combine matches the reference's
    per-expert index_add (ascending expert order, weight cast to the
    output dtype) bit for bit."""
    from spider_moe_amd.dispatch import dispatch_expert_ffn
    say("dispatch_expert_fn", dtype, n, h, e, k)
    g = torch.Generator().manual_seed(n + h)
    msg = torch.randn(2, n, h, generator=g).to(dtype)
    ti = torch.randint(0, e, (2, n, k), generator=g)
    ti[0, 0] = torch.tensor([2] * (k - 1) + [1])  # duplicate slots merge
    tw = torch.rand(2, n, k, generator=g)
    tw[0, 1, 0] = 0.0
    seen = []

    def fn(eid, x):
        seen.append(eid)
        return x * float(eid + 1) + 0.25

    got = dispatch_expert_ffn(msg.to(dev), ti.to(dev), tw.to(dev), w_up=None, b_up=None,
                              w_down=None, b_down=None, num_experts=e, expert_fn=fn).cpu()
    assert seen == sorted(set(seen)) and len(seen) >= 2
    want = OF.dispatch_ffn(msg, ti, tw, e, fn)
    assert got.dtype == dtype and torch.equal(got, want)


# ------------------------------------------- host ABI (spider_kernels.h) ----
def _host():
    from spider_moe_amd.native_compat import HostKernels
    return HostKernels()


def test_host_abi_known_answers():
    """The reference's own C++ checks (kernels/tests/test_kernels.cpp:7-18,
    test_phase1_1.cpp:8-57, test_phase1_2.cpp:7-45, test_phase1_3.cpp:7-52)
    through the host entry points on the GPU."""
    say("host abi known answers")
    hk = _host()
    assert hk.backend == "hip-gfx950"
    w, i = hk.router(np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float32), np.zeros((1, 4), np.float32), 2)
    assert i.tolist() == [[3, 2], [0, 1]] and np.allclose(w.sum(-1), 1, atol=1e-6)
    h = (0.1 * np.arange(1, 9, dtype=np.float32)).reshape(2, 4)
    we = np.stack([np.eye(4, dtype=np.float32)] * 3)
    assert np.allclose(hk.edge_project(h, we), np.repeat(h[:, None], 3, axis=1), atol=1e-5)
    m = hk.graph_v2(np.array([[[1, 0], [0, 2]]], np.float32), np.array([0, 1, 1]), np.array([1]),
                    np.array([0.5], np.float32), np.array([[0]]), 2)
    assert np.allclose(m, [[0, 1]], atol=1e-6)
    idx, wt = hk.edge_topk(np.array([[[0, 1, 2], [3, 0, 1], [0, 0, 1]]], np.float32), 2)
    assert idx[0, 0].tolist() == [2, 1] and abs(wt[0, 0].sum() - 1) < 1e-5
    m = hk.graph_dynamic(np.array([[[1, 0], [0, 4]]], np.float32), np.array([[[1], [0]]]),
                         np.array([[[0.5], [1.0]]], np.float32), np.array([[0]]), 2, 1)
    assert np.allclose(m, [[0, 2]], atol=1e-5)
    wg = np.zeros((4, 3), np.float32)
    wg[1, 0] = wg[2, 0] = 5
    lg = hk.edge_generator(np.array([[1, 0]], np.float32), np.zeros(1, np.float32), wg, 2)
    assert lg.reshape(-1)[1] > lg.reshape(-1)[0]
    wg = np.zeros((4, 2), np.float32)
    wg[1, 0] = wg[2, 0] = 3
    idx, wt = hk.edge_topk(hk.edge_generator(np.array([[1, 0]], np.float32),
                                             np.zeros(0, np.float32), wg, 2), 1)
    assert idx[0, 0, 0] == 1 and abs(wt[0, 0, 0] - 1) < 1e-5
    wg = np.zeros((4, 2), np.float32)
    wg[1, 0] = 2
    m = hk.graph_from_generator(np.array([[1, 0]], np.float32), np.zeros(0, np.float32), wg,
                                np.stack([np.eye(2, dtype=np.float32)] * 2), np.array([[0]]), 2, 1)
    assert np.isfinite(m).all()
    out, mask, *_ = hk.moe_loop_step(
        np.full((1, 4), 0.05, np.float32), np.full((1, 4), 0.01, np.float32), 0,
        router_w=np.full((4, 2), 0.02, np.float32), loop_bias=np.zeros(2, np.float32),
        W_up=np.full((2, 4, 4), 0.01, np.float32), W_down=np.full((2, 4, 4), 0.01, np.float32),
        ln_weight=np.ones(4, np.float32), ln_bias=np.zeros(4, np.float32), top_k=1, alpha=1.0,
        beta=0.0, csr=(np.array([0, 1, 1]), np.array([0]), np.ones(1, np.float32)),
        W_edge=np.stack([np.eye(4, dtype=np.float32)] * 2), exit_proj=np.full(4, 0.1, np.float32),
        exit_threshold=0.99)
    assert np.isfinite(out).all()
    with pytest.raises(RuntimeError, match="spider_expert_grouped_gemm_f32 failed: 2"):
        hk.expert_ffn(np.zeros((1, 4), np.float32), np.array([[3]]), np.ones((1, 1), np.float32),
                      np.zeros((2, 4, 4), np.float32), np.zeros((2, 4, 4), np.float32), 2)


@pytest.mark.parametrize("b,h,e,m,k", [(6, 24, 8, 3, 2), (4, 64, 100, 5, 4), (3, 32, 256, 4, 8)])
def test_host_abi_dynamic_edges_match_oracle(b, h, e, m, k):
    """Edge projection, generator, graph v2 and the dynamic pass are the
    scalar library's float / double operations in its order: exact.  Edge
    top-m indices exact, weights within expf's ulps; E up to 256."""
    say("host abi dynamic", b, h, e, m, k)
    hk = _host()
    r = _rng(e + h)
    x = r.standard_normal((b, h)).astype(np.float32)
    we = (r.standard_normal((e, h, h)) / np.sqrt(h)).astype(np.float32)
    proj = hk.edge_project(x, we)
    assert np.array_equal(proj, ON.edge_project(x, we))
    d = 3
    wg = (r.standard_normal((e * e, h + d)) / np.sqrt(h)).astype(np.float32)
    emb = r.standard_normal(d).astype(np.float32)
    lg = hk.edge_generator(x, emb, wg, e)
    assert np.array_equal(lg, ON.edge_generator(x, emb, wg))
    lg[0, 1, :4] = lg[0, 1, 5]  # ties: first index
    lg[0, 2, :] = -np.inf
    lg[0, 2, 3] = 1.0  # one candidate, then none
    idx, wt = hk.edge_topk(lg, m)
    io, wo = ON.edge_topk(lg, m)
    assert np.array_equal(idx, io)
    fin = np.isfinite(wo)
    assert np.allclose(wt[fin], wo[fin], rtol=1e-5, atol=1e-7)
    asg = r.integers(-1, e, (b, k)).astype(np.int32)
    asg[0, 0] = 1
    ok = (idx >= 0).all(-1)  # sources whose picks are all valid
    asg_ok = np.where(np.take_along_axis(ok, np.maximum(asg, 0), 1) | (asg < 0), asg, -1)
    got = hk.graph_dynamic(proj, idx, wt, asg_ok, e, m)
    assert np.array_equal(got, ON.graph_dynamic(proj, idx, wt, asg_ok))
    rp = np.concatenate([[0], np.cumsum(r.integers(0, 3, e))]).astype(np.int32)
    nnz = int(rp[-1])
    ci = r.integers(0, e, nnz).astype(np.int32)
    ew = r.random(2 * nnz).astype(np.float32)
    for loop in (0, 1):
        got = hk.graph_v2(proj, rp, ci, ew, asg, e, loop)
        assert np.array_equal(got, ON.graph_v2(proj, rp, ci, ew, asg, nnz=nnz, loop_idx=loop))
    lgr = r.standard_normal((b * 7, e)).astype(np.float32)
    bias = (0.1 * r.standard_normal((2, e))).astype(np.float32)
    w, i = hk.router(lgr, bias, k, 1)
    wo, io = ON.router(lgr, bias[1], k)
    assert np.array_equal(i, io) and np.allclose(w, wo, rtol=1e-5, atol=1e-7)


def test_host_abi_loop_step_matches_oracle():
    say("host abi loop step")
    hk = _host()
    r = _rng(31)
    b, h, e, k, u = 64, 128, 16, 2, 96
    x, x0 = (r.standard_normal((b, h)).astype(np.float32) for _ in range(2))
    rw = (r.standard_normal((h, e)) / np.sqrt(h)).astype(np.float32)
    bias = (0.1 * r.standard_normal((3, e))).astype(np.float32)
    wu = (r.standard_normal((e, h, u)) / np.sqrt(h)).astype(np.float32)
    wd = (r.standard_normal((e, u, h)) / np.sqrt(u)).astype(np.float32)
    we = (r.standard_normal((e, h, h)) / np.sqrt(h)).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(h)).astype(np.float32)
    gb = (0.1 * r.standard_normal(h)).astype(np.float32)
    proj = (r.standard_normal(h) / np.sqrt(h)).astype(np.float32)
    rp, ci = _csr(e, r)
    ew = r.random(3 * len(ci)).astype(np.float32)
    for csr, wedge in (((rp, ci, ew), we), (None, None)):
        hn, mask, asg, route, msgs = hk.moe_loop_step(
            x, x0, 2, router_w=rw, loop_bias=bias, W_up=wu, W_down=wd, ln_weight=g, ln_bias=gb,
            top_k=k, alpha=0.5, beta=0.1, csr=csr, W_edge=wedge, exit_proj=proj,
            exit_threshold=0.5)
        wn, _, wa, wr, wm = ON.loop_step(x, x0, k, rw, bias[2], wu, wd, g, gb, 0.5, 0.1, 1e-5,
                                         csr=csr, w_edge=wedge, loop_idx=2)
        assert np.array_equal(asg, wa) and np.allclose(route, wr, rtol=1e-5, atol=1e-7)
        assert np.allclose(msgs, wm, rtol=1e-5, atol=1e-5)
        assert np.allclose(hn, wn, rtol=1e-4, atol=1e-4)
        _, conf = ON.exit_mask(wn, proj, 0.5)
        far = np.abs(conf - 0.5) > 1e-4
        assert np.array_equal(mask[far], (conf[far] > 0.5).astype(np.uint8))


def test_host_abi_matches_the_compiled_scalar_library():
    """Where oracle/_ref (the reference's scalar library compiled from its
    sources) is present, the same calls on both libraries agree."""
    from oracle import ref as R
    if not R.available():
        pytest.skip("oracle/_ref not built")
    say("host abi vs scalar library")
    hk = _host()
    r = _rng(41)
    b, h, e, m, k, u = 5, 32, 8, 3, 2, 40
    x = r.standard_normal((b, h)).astype(np.float32)
    we = (0.3 * r.standard_normal((e, h, h))).astype(np.float32)
    rc, pr = R.edge_project_f32(x, we)
    assert rc == 0 and np.array_equal(hk.edge_project(x, we), pr)
    wg = (0.3 * r.standard_normal((e * e, h + 2))).astype(np.float32)
    emb = r.standard_normal(2).astype(np.float32)
    rc, lr = R.edge_generator_f32(x, emb, wg)
    assert rc == 0 and np.array_equal(hk.edge_generator(x, emb, wg, e), lr)
    rc, ir, wr = R.edge_topk_f32(lr, m)
    idx, wt = hk.edge_topk(lr, m)
    assert np.array_equal(idx, ir) and np.allclose(wt, wr, rtol=1e-5)
    asg = r.integers(-1, e, (b, k)).astype(np.int32)
    rc, gr = R.graph_dynamic_f32(pr, ir, wr, asg)
    assert rc == 0 and np.array_equal(hk.graph_dynamic(pr, ir, wr, asg, e, m), gr)
    wu = (0.2 * r.standard_normal((e, h, u))).astype(np.float32)
    wd = (0.2 * r.standard_normal((e, u, h))).astype(np.float32)
    rw = r.random((b, k)).astype(np.float32)
    rc, er = R.expert_grouped_gemm_f32(x, asg, rw, wu, wd)
    assert rc == 0 and np.allclose(hk.expert_ffn(x, asg, rw, wu, wd, e), er, rtol=1e-4, atol=1e-5)
