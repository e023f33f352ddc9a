"""Pins for oracle/native.py (the reference's native loop kernels) and
oracle/forge.py (the Forge surfaces), and the .spiderw format, on the CPU.

oracle/native.py is checked against oracle/_ref, the reference's scalar
library compiled from its own sources: bit for bit where both run the same
float operations (graph, epilogue, loop-step logits), within an ulp-level
tolerance where a libm function enters (exp in the router, tanh in the
GELU), and against the reference's known answers
(kernels/tests/test_kernels.cpp:7-18)."""
import numpy as np
import pytest
import torch

from oracle import forge as OF
from oracle import native as ON
from oracle import quant as OQ
from oracle import ref as R

needs_ref = pytest.mark.skipif(not R.available(), reason="oracle/_ref not built")
rng = np.random.default_rng(7)


def _case(b=6, h=32, e=8, k=2, u=24):
    return dict(h=rng.standard_normal((b, h)).astype(np.float32),
                x0=rng.standard_normal((b, h)).astype(np.float32),
                logits=rng.standard_normal((b, e)).astype(np.float32),
                bias=(0.1 * rng.standard_normal((3, e))).astype(np.float32),
                w_up=(0.2 * rng.standard_normal((e, h, u))).astype(np.float32),
                w_down=(0.2 * rng.standard_normal((e, u, h))).astype(np.float32),
                router_w=(0.3 * rng.standard_normal((h, e))).astype(np.float32),
                gamma=(1 + 0.1 * rng.standard_normal(h)).astype(np.float32),
                beta=(0.1 * rng.standard_normal(h)).astype(np.float32), k=k)


def test_native_router_known_answer():
    """kernels/tests/test_kernels.cpp:7-18: logits {1,2,3,4} and {4,3,2,1},
    k = 2 -> experts {3, 2} and {0, 1}, weights summing to 1."""
    w, i = ON.router(np.array([[1, 2, 3, 4], [4, 3, 2, 1]], np.float32), np.zeros(4, np.float32), 2)
    assert i.tolist() == [[3, 2], [0, 1]]
    assert np.allclose(w.sum(-1), 1.0, atol=1e-6)
    assert np.allclose(w[0], [np.exp(1) / (1 + np.exp(1)), 1 / (1 + np.exp(1))], rtol=1e-6)


@needs_ref
def test_native_router_matches_scalar_library():
    c = _case(b=40, e=16, k=4)
    for loop in range(3):
        rc, wr, ir = R.router_f32(c["logits"], c["bias"], 4, loop)
        assert rc == 0
        w, i = ON.router(c["logits"], c["bias"][loop], 4)
        assert np.array_equal(i, ir)
        assert np.allclose(w, wr, rtol=2e-6, atol=1e-7)


@needs_ref
def test_native_graph_v1_matches_scalar_library_bit_for_bit():
    c = _case(b=5, h=16, e=6, k=2)
    rp = np.array([0, 2, 3, 5, 5, 7, 8], np.int32)
    ci = np.array([1, 2, 0, 3, 4, 5, 0, 1], np.int32)
    ew = rng.random(8 * 2).astype(np.float32)  # two loops of edge weights
    asg = np.array([[0, 2], [1, 5], [3, 4], [2, 2], [5, 0]], np.int32)
    rw = rng.random((5, 2)).astype(np.float32)
    for loop in (0, 1):
        rc, ref = R.graph_message_passing_f32(c["h"][:5, :16], rp, ci, ew, asg, rw, loop)
        assert rc == 0
        got = ON.graph_v1(c["h"][:5, :16], rp, ew, asg, rw, nnz=8, loop_idx=loop)
        assert np.array_equal(got, ref)


@needs_ref
def test_native_experts_match_scalar_library():
    c = _case(b=5, h=32, e=4, k=2, u=24)
    asg = np.array([[0, 1], [3, 3], [2, 0], [1, -1], [3, 2]], np.int32)
    rw = rng.random((5, 2)).astype(np.float32)
    rc, ref = R.expert_grouped_gemm_f32(c["h"][:5], asg, rw, c["w_up"][:4], c["w_down"][:4])
    assert rc == 0
    got = ON.experts(c["h"][:5], asg, rw, c["w_up"][:4], c["w_down"][:4])
    assert np.allclose(got, ref, rtol=1e-5, atol=1e-6)


@needs_ref
def test_native_epilogue_and_exit_match_scalar_library():
    c = _case(b=8, h=48)
    d = rng.standard_normal((8, 48)).astype(np.float32)
    rc, ref = R.loop_epilogue_f32(c["h"][:, :48], d, c["x0"][:, :48], 0.5, 0.1, c["gamma"][:48],
                                  c["beta"][:48], 1e-5)
    assert rc == 0
    got = ON.epilogue(c["h"][:, :48], d, c["x0"][:, :48], 0.5, 0.1, c["gamma"][:48],
                      c["beta"][:48], 1e-5)
    assert np.array_equal(got, ref)
    proj = (0.2 * rng.standard_normal(48)).astype(np.float32)
    for thr in (0.3, 0.5, 0.7):
        rc, mref = R.early_exit_f32(got, proj, thr)
        mask, conf = ON.exit_mask(got, proj, thr)
        far = np.abs(conf - thr) > 1e-6
        assert rc == 0 and np.array_equal(mask[far], mref[far])


@needs_ref
def test_native_loop_step_matches_scalar_library():
    """scalar spider_moe_loop_step_f32 with no graph (messages = h) and an
    exit head; and the reference's exit-mask zeroing without one."""
    c = _case(b=7, h=32, e=8, k=2, u=24)
    proj = (0.2 * rng.standard_normal(32)).astype(np.float32)
    for loop, ep in ((1, proj), (2, None)):
        rc, hn, m, asg, route = R.moe_loop_step_f32(c["h"][:7], c["x0"][:7], 2, loop, c["router_w"],
                                                   c["bias"], c["w_up"], c["w_down"], c["gamma"][:32],
                                                   c["beta"][:32], 0.5, 0.1, 1e-5, ep, 0.5)
        assert rc == 0
        got, mg, ag, rg, _ = ON.loop_step(c["h"][:7], c["x0"][:7], 2, c["router_w"], c["bias"][loop],
                                          c["w_up"], c["w_down"], c["gamma"][:32], c["beta"][:32],
                                          0.5, 0.1, 1e-5, exit_proj=ep, threshold=0.5)
        assert np.array_equal(ag, asg)
        assert np.allclose(rg, route, rtol=2e-6)
        assert np.allclose(got, hn, rtol=1e-5, atol=1e-5)
        assert np.array_equal(mg, m)


def test_planted_native_mistake_is_caught():
    """A graph that forgets the route weight, or an epilogue with alpha and
    beta swapped, differs from the oracle."""
    c = _case(b=3, h=16, e=4, k=2)
    rp = np.array([0, 1, 2, 3, 4], np.int32)
    asg = np.array([[0, 1], [2, 3], [1, 2]], np.int32)
    rw = np.full((3, 2), 0.5, np.float32)
    ew = np.ones(4, np.float32)
    good = ON.graph_v1(c["h"][:3, :16], rp, ew, asg, rw)
    bad = ON.graph_v1(c["h"][:3, :16], rp, ew, asg, np.ones_like(rw))
    assert not np.allclose(good, bad)
    d = rng.standard_normal((3, 16)).astype(np.float32)
    e1 = ON.epilogue(c["h"][:3, :16], d, c["x0"][:3, :16], 0.5, 0.1, np.ones(16, np.float32),
                     np.zeros(16, np.float32), 1e-5)
    e2 = ON.epilogue(c["h"][:3, :16], d, c["x0"][:3, :16], 0.1, 0.5, np.ones(16, np.float32),
                     np.zeros(16, np.float32), 1e-5)
    assert not np.allclose(e1, e2)


# ------------------------------------------------------------- forge ----
def test_select_route_known_answer():
    """forge/select/api.py:28-40: top-k on the logits, softmax over k."""
    w, i = OF.select_route(torch.tensor([[1.0, 3.0, 2.0, 0.0]]), 2)
    assert i.tolist() == [[1, 2]]
    e = float(np.exp(1.0))
    assert torch.allclose(w, torch.tensor([[e / (1 + e), 1 / (1 + e)]], dtype=torch.float32),
                          atol=1e-7)


def test_fp8_per_tensor_scale_and_codes():
    """scale = amax / 448 over the whole tensor; codes decode (e4m3 table)
    to values within half an e4m3 step of w / scale; the largest |w| maps
    to 448 exactly."""
    w = torch.randn(24, 40, generator=torch.Generator().manual_seed(3)) * 0.05
    codes, scale = OF.fp8_quantize_per_tensor(w)
    assert float(scale) == pytest.approx(float(w.abs().max()) / 448.0, rel=1e-7)
    dec = torch.from_numpy(OQ.fp8_e4m3_decode(codes.view(torch.uint8).numpy()))
    assert float(dec.abs().max()) == 448.0
    q = w / scale
    assert bool(((dec - q).abs() <= q.abs() * 2 ** -4 + 2 ** -10).all())


def test_fp8_linear_quantize_input_known_answer_and_scale_invariance():
    """quantize_input (forge/gemm/fp8.py:49-51): inputs already on the e4m3
    grid of their own scale (amax 448 -> scale 1) pass unchanged, so the
    product is exact; a power-of-two multiple of x gives the same codes with
    the scale times that power, and the output scales with it; dropping the
    input scale (multiplying the raw codes) misses by the scale."""
    x = torch.tensor([[448.0, -224.0, 1.0, 0.0, 0.5, -3.0, 0.015625, 2.0 ** -9]])
    w = torch.tensor([[1.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                      [0.0, 1.0, 1.0, 0.0, 0.0, 0.0, 0.0, 0.0],
                      [0.0, 0.0, 0.0, 0.0, 1.0, 1.0, 1.0, 1.0]]) * 448.0
    xc, xs = OF.fp8_quantize_per_tensor(x)
    assert float(xs) == 1.0
    assert torch.equal(xc.float(), x)
    got = OF.fp8_linear(x, w, quantize_input=True)
    want = torch.tensor([[448.0 * 448.0, -223.0 * 448.0,
                          (0.5 - 3.0 + 0.015625 + 2.0 ** -9) * 448.0]])
    assert torch.equal(got, want)
    g = torch.Generator().manual_seed(12)
    xr = torch.randn(6, 40, generator=g) * 0.3
    wr = torch.randn(10, 40, generator=g) * 0.05
    c1, s1 = OF.fp8_quantize_per_tensor(xr)
    c2, s2 = OF.fp8_quantize_per_tensor(xr * 8.0)
    assert torch.equal(c1.view(torch.uint8), c2.view(torch.uint8)) and float(s2) == 8.0 * float(s1)
    y1 = OF.fp8_linear(xr, wr, quantize_input=True)
    y2 = OF.fp8_linear(xr * 8.0, wr, quantize_input=True)
    assert torch.allclose(y2, 8.0 * y1, rtol=1e-6, atol=1e-7)
    # the quantized input stays within e4m3 rounding of the exact product
    exact = xr @ (OF.fp8_quantize_per_tensor(wr)[0].float() * OF.fp8_quantize_per_tensor(wr)[1]).t()
    assert (y1 - exact).abs().max() <= 0.07 * exact.abs().max()
    wc, ws = OF.fp8_quantize_per_tensor(wr)
    raw = c1.float() @ (wc.float() * ws).t()  # planted: no input scale
    assert (raw - y1).abs().max() > 10 * (y1 - exact).abs().max()


def test_dispatch_ffn_oracle_matches_per_token_loop():
    """The dispatch combine equals, per token, the sum over its experts in
    ascending order of expert_fn(e, x_t) times the merged weight (duplicate
    slots merged, weights <= 0 dropped)."""
    g = torch.Generator().manual_seed(4)
    msg = torch.randn(10, 8, generator=g)
    ti = torch.randint(0, 5, (10, 3), generator=g)
    ti[0] = torch.tensor([2, 2, 1])  # duplicate slot
    tw = torch.rand(10, 3, generator=g)
    tw[1, 0] = 0.0
    fn = lambda e, x: x * float(e + 1) + 0.25  # noqa: E731
    got = OF.dispatch_ffn(msg, ti, tw, 5, fn)
    want = torch.zeros_like(msg)
    for t in range(10):
        merged = {}
        for s in range(3):
            merged[int(ti[t, s])] = merged.get(int(ti[t, s]), 0.0) + float(tw[t, s])
        for e in sorted(merged):
            if merged[e] > 0:
                want[t] += fn(e, msg[t:t + 1])[0] * merged[e]
    assert torch.allclose(got, want, atol=1e-6)


# ----------------------------------------------------------- spiderw ----
def test_spiderw_roundtrip(tmp_path):
    from spider_moe_amd.spiderw import SpiderWMeta, load_spiderw, write_spiderw
    meta = SpiderWMeta(version=1, flags=2 | 4, vocab_size=32, hidden_size=16, num_heads=2,
                       num_experts=4, top_k=2, edges_per_expert=2, num_loops=3,
                       expert_ffn_size=24)
    t = {"token_emb": rng.standard_normal((32, 16)).astype(np.float32),
         "router": rng.standard_normal((16, 4)).astype(np.float32),
         "expert_up": rng.standard_normal((4, 16, 24)).astype(np.float16),
         "csr_row_ptr": np.array([0, 1, 2, 3, 4], np.int32),
         "csr_col_idx": np.array([1, 2, 3, 0], np.int32),
         "csr_edge_w": np.ones(4, np.float32),
         "my_extra": np.arange(6, dtype=np.int32).reshape(2, 3)}
    p = tmp_path / "m.spiderw"
    write_spiderw(p, meta, t)
    raw = p.read_bytes()
    assert raw[:8] == b"SPIDERW1"
    b = load_spiderw(p)
    assert b.meta == meta and b.meta.has_csr and b.meta.tied_embeddings
    for name, a in t.items():
        assert b.tensors[name].dtype == a.dtype and np.array_equal(b.tensors[name], a), name
    assert np.array_equal(b.tensors["lm_head"], t["token_emb"])  # tied
    assert np.array_equal(b.csr["col_idx"], t["csr_col_idx"])
    # a truncated trailing section ends the read, the earlier ones stay
    p2 = tmp_path / "cut.spiderw"
    p2.write_bytes(raw[:-5])
    b2 = load_spiderw(p2)
    assert "token_emb" in b2.tensors and "my_extra" not in b2.tensors
    with pytest.raises(ValueError):
        load_spiderw_bytes = tmp_path / "bad.spiderw"
        load_spiderw_bytes.write_bytes(b"NOTSPIDR" + raw[8:])
        load_spiderw(load_spiderw_bytes)


# ---------------------------------------------- dynamic-edge functions ----
def test_dynamic_edge_known_answers():
    """kernels/tests/test_phase1_1.cpp:8-33, test_phase1_2.cpp:7-31,
    test_phase1_3.cpp:7-33."""
    h = (0.1 * np.arange(1, 9, dtype=np.float32)).reshape(2, 4)
    w = np.zeros((3, 4, 4), np.float32)
    for e in range(3):
        w[e] = np.eye(4, dtype=np.float32)
    p = ON.edge_project(h, w)
    assert np.allclose(p, np.repeat(h[:, None, :], 3, axis=1), atol=1e-7)
    m = ON.graph_v2(np.array([[[1, 0], [0, 2]]], np.float32), np.array([0, 1, 1]), np.array([1]),
                    np.array([0.5], np.float32), np.array([[0]]))
    assert np.allclose(m, [[0, 1]])
    idx, wt = ON.edge_topk(np.array([[[0, 1, 2], [3, 0, 1], [0, 0, 1]]], np.float32), 2)
    assert idx[0, 0].tolist() == [2, 1] and abs(wt[0, 0].sum() - 1) < 1e-6
    assert idx[0, 2].tolist() == [2, 0]  # ties go to the lower index
    m = ON.graph_dynamic(np.array([[[1, 0], [0, 4]]], np.float32), np.array([[[1], [0]]]),
                         np.array([[[0.5], [1.0]]], np.float32), np.array([[0]]))
    assert np.allclose(m, [[0, 2]])
    wg = np.zeros((4, 3), np.float32)
    wg[1, 0] = wg[2, 0] = 5
    lg = ON.edge_generator(np.array([[1, 0]], np.float32), np.zeros(1, np.float32), wg)
    assert lg.reshape(-1)[1] > lg.reshape(-1)[0]
    wg = np.zeros((4, 2), np.float32)
    wg[1, 0] = wg[2, 0] = 3
    idx, wt = ON.edge_topk(ON.edge_generator(np.array([[1, 0]], np.float32),
                                             np.zeros(0, np.float32), wg), 1)
    assert idx[0, 0, 0] == 1 and abs(wt[0, 0, 0] - 1) < 1e-6


def test_edge_topk_without_candidates():
    """All remaining logits -inf (or NaN): the pick is (-1, -inf), as the
    scalar loop leaves it."""
    g = np.full((1, 2, 2), -np.inf, np.float32)
    g[0, 0, 1] = 0.5
    g[0, 1, 0] = np.nan
    idx, _ = ON.edge_topk(g, 2)
    assert idx[0, 0].tolist() == [1, -1] and idx[0, 1].tolist() == [-1, -1]


@needs_ref
def test_dynamic_edge_functions_match_scalar_library():
    r = np.random.default_rng(21)
    b, h, e, m, k, d = 6, 24, 8, 3, 2, 5
    x = r.standard_normal((b, h)).astype(np.float32)
    we = (0.3 * r.standard_normal((e, h, h))).astype(np.float32)
    rc, pr = R.edge_project_f32(x, we)
    assert rc == 0 and np.array_equal(ON.edge_project(x, we), pr)
    wg = (0.3 * r.standard_normal((e * e, h + d))).astype(np.float32)
    emb = r.standard_normal(d).astype(np.float32)
    rc, lr = R.edge_generator_f32(x, emb, wg)
    lo = ON.edge_generator(x, emb, wg)
    assert rc == 0 and np.array_equal(lo, lr)
    lo[0, 1, :3] = lo[0, 1, 3]  # ties
    rc, ir, wr = R.edge_topk_f32(lo, m)
    io, wo = ON.edge_topk(lo, m)
    assert rc == 0 and np.array_equal(io, ir) and np.allclose(wo, wr, rtol=2e-6)
    asg = r.integers(-1, e, (b, k)).astype(np.int32)
    rc, gr = R.graph_dynamic_f32(pr, ir, wr, asg)
    assert rc == 0 and np.array_equal(ON.graph_dynamic(pr, ir, wr, asg), gr)
    rp = np.array([0, 2, 3, 3, 5, 6, 8, 9, 10], np.int32)
    ci = r.integers(0, e, 10).astype(np.int32)
    ew = r.random(20).astype(np.float32)
    for loop in (0, 1):
        rc, vr = R.graph_v2_f32(pr, rp, ci, ew, asg, loop)
        assert rc == 0
        assert np.array_equal(ON.graph_v2(pr, rp, ci, ew, asg, nnz=10, loop_idx=loop), vr)


@needs_ref
def test_loop_step_with_edge_values_matches_scalar_library():
    r = np.random.default_rng(22)
    b, h, e, k, u = 5, 16, 6, 2, 24
    x, x0 = (r.standard_normal((b, h)).astype(np.float32) for _ in range(2))
    rw = (0.3 * r.standard_normal((h, e))).astype(np.float32)
    bias = (0.1 * r.standard_normal((2, e))).astype(np.float32)
    wu = (0.2 * r.standard_normal((e, h, u))).astype(np.float32)
    wd = (0.2 * r.standard_normal((e, u, h))).astype(np.float32)
    we = (0.3 * r.standard_normal((e, h, h))).astype(np.float32)
    g = (1 + 0.1 * r.standard_normal(h)).astype(np.float32)
    gb = (0.1 * r.standard_normal(h)).astype(np.float32)
    rp = np.array([0, 1, 3, 3, 4, 6, 7], np.int32)
    ci = r.integers(0, e, 7).astype(np.int32)
    ew = r.random(14).astype(np.float32)
    rc, hn, mk, asg, route = R.moe_loop_step_f32(x, x0, k, 1, rw, bias, wu, wd, g, gb, 0.5, 0.1,
                                                 1e-5, None, 0.5, csr=(rp, ci, ew), w_edge=we)
    assert rc == 0
    got, mg, ag, rg, _ = ON.loop_step(x, x0, k, rw, bias[1], wu, wd, g, gb, 0.5, 0.1, 1e-5,
                                      csr=(rp, ci, ew), w_edge=we, loop_idx=1)
    assert np.array_equal(ag, asg) and np.allclose(rg, route, rtol=2e-6)
    assert np.allclose(got, hn, rtol=1e-5, atol=1e-5) and not mg.any() and not mk.any()


def test_planted_dynamic_edge_mistakes_are_caught():
    """A projection with W_edge transposed, or a top-m without the
    softmax, differs from the oracle."""
    r = np.random.default_rng(23)
    x = r.standard_normal((2, 8)).astype(np.float32)
    we = r.standard_normal((3, 8, 8)).astype(np.float32)
    assert not np.allclose(ON.edge_project(x, we), ON.edge_project(x, we.transpose(0, 2, 1)))
    g = r.standard_normal((1, 4, 4)).astype(np.float32)
    _, w = ON.edge_topk(g, 2)
    assert np.allclose(w.sum(-1), 1, atol=1e-6) and not np.allclose(w, np.sort(g, -1)[..., ::-1][..., :2])
