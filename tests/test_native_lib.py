"""CPU checks of libsmoe.so: it loads without a GPU, exports every entry
point include/smoe.h declares, and its host-side argument validation and
workspace layout behave (no kernel is launched here)."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "smoe.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"SMOE_API\s+[\w\s\*]+?\b(smoe_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def nat():
    from spider_moe_amd import _native
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail("libsmoe.so is not built (run __graft_entry__.build())")
    _native.lib()
    return _native


def test_exports_every_declared_symbol(nat):
    syms = declared_symbols()
    assert len(syms) >= 14
    handle = ctypes.CDLL(nat.LIB_PATH)
    for s in syms:
        assert hasattr(handle, s), s
    # and the Python binding covers exactly the declared set
    assert set(nat.SIGNATURES) == set(syms)


def test_exports_the_reference_device_abi(nat):
    """include/spider_cuda.h: the reference's device ABI names
    (kernels/include/spider_cuda.h:8-44), exported by libsmoe.so."""
    text = open(os.path.join(ROOT, "include", "spider_cuda.h")).read()
    syms = sorted(set(re.findall(r"SPIDER_CUDA_API\s+[\w\s\*]+?\b(spider_cuda_\w+)\s*\(", text)))
    assert syms == sorted(["spider_cuda_router_f32", "spider_cuda_graph_message_passing_f32",
                           "spider_cuda_expert_grouped_gemm_f32",
                           "spider_cuda_expert_workspace_bytes",
                           "spider_cuda_expert_grouped_gemm_v2_f32",
                           "spider_cuda_loop_epilogue_f32", "spider_cuda_early_exit_f32",
                           "spider_cuda_moe_loop_step_f32",
                           # device forms of the dynamic-edge host functions
                           "spider_cuda_edge_project_f32",
                           "spider_cuda_graph_message_passing_v2_f32",
                           "spider_cuda_edge_topk_f32",
                           "spider_cuda_graph_message_passing_dynamic_f32",
                           "spider_cuda_edge_generator_f32"])
    handle = ctypes.CDLL(nat.LIB_PATH)
    for s in syms:
        assert hasattr(handle, s), s
    assert set(nat.SPIDER_CUDA_SIGNATURES) == set(syms)
    lib = nat.lib()
    assert lib.spider_cuda_expert_workspace_bytes(4, 2, 8) == 4 * 2 * 8 * 4
    assert lib.spider_cuda_expert_workspace_bytes(0, 2, 8) == 0
    # argument checks return 1 before any launch
    assert lib.spider_cuda_router_f32(None, None, 1, 4, 2, 0, None, None, None) == 1
    assert lib.spider_cuda_router_f32(1, 1, 1, 257, 2, 0, 1, 1, None) == 1  # E > 256
    assert lib.spider_cuda_early_exit_f32(None, None, 1, 4, 0.5, None, None) == 1
    assert lib.spider_cuda_edge_topk_f32(1, 1, 4, 5, 1, 1, None) == 1  # M > E


def test_exports_the_reference_host_abi(nat):
    """include/spider_kernels.h: the reference's host ABI names of the MoE
    loop (kernels/include/spider_kernels.h:26-121, 148-149); the argument
    and index checks run on the host before any device work, so they are
    exercised here without a GPU; the f16 entries return -2 like the
    reference's stubs."""
    import numpy as np
    text = open(os.path.join(ROOT, "include", "spider_kernels.h")).read()
    syms = sorted(set(re.findall(r"SPIDER_API\s+[\w\s\*]+?\b(spider_\w+)\s*\(", text)))
    assert set(nat.SPIDER_HOST_SIGNATURES) == set(syms)
    assert {"spider_router_f32", "spider_edge_topk_f32", "spider_graph_message_passing_dynamic_f32",
            "spider_expert_grouped_gemm_f32", "spider_loop_epilogue_f32", "spider_early_exit_f32",
            "spider_moe_loop_step_f32"} <= set(syms)
    alias = os.path.join(os.path.dirname(nat.LIB_PATH), "libspider_kernels.so")
    assert os.path.realpath(alias) == os.path.realpath(nat.LIB_PATH)
    handle = ctypes.CDLL(alias)
    for s in syms:
        assert hasattr(handle, s), s
    lib = nat.lib()
    assert lib.spider_backend_name() == b"hip-gfx950" and lib.spider_backend_caps() & 1
    for f16 in ("spider_router_f16", "spider_graph_message_passing_f16",
                "spider_expert_grouped_gemm_f16", "spider_loop_epilogue_f16"):
        args = [None if t is ctypes.c_void_p else t(0)
                for t in nat.SPIDER_HOST_SIGNATURES[f16][1]]
        assert getattr(lib, f16)(*args) == -2
    z = np.zeros(64, np.float32)
    zi = np.zeros(64, np.int32)
    p = lambda a: a.ctypes.data  # noqa: E731
    assert lib.spider_router_f32(p(z), p(z), 2, 4, 5, 0, p(z), p(zi)) == 1  # K > E
    assert lib.spider_router_f32(None, p(z), 2, 4, 2, 0, p(z), p(zi)) == 1
    assert lib.spider_loop_epilogue_f32(p(z), p(z), p(z), 1, 4, 1.0, 0.0, p(z), p(z), 0.0,
                                        p(z)) == 1  # eps <= 0
    assert lib.spider_edge_topk_f32(p(z), 1, 2, 3, p(zi), p(z)) == 1  # M > E
    # a CSR that does not end at nnz, then a selected source >= E
    rp = np.array([0, 1, 1], np.int32)
    ci = np.array([1], np.int32)
    asg = np.array([0, 2], np.int32)
    assert lib.spider_graph_message_passing_f32(p(z), 2, 4, 2, 1, p(rp), p(ci), p(z), 2, 0,
                                                p(asg), p(z), p(z)) == 1
    assert lib.spider_graph_message_passing_f32(p(z), 2, 4, 2, 1, p(rp), p(ci), p(z), 1, 0,
                                                p(asg), p(z), p(z)) == 2
    ci_bad = np.array([5], np.int32)  # destination outside [0, E) of a selected source
    asg0 = np.array([0, -1], np.int32)
    assert lib.spider_graph_message_passing_v2_f32(p(z), 2, 4, 2, 1, p(rp), p(ci_bad), p(z), 1,
                                                   0, p(asg0), p(z)) == 2
    eidx = np.array([0, 7, 0, 0], np.int32)  # [B=1, E=2, M=2]: source 0 points at 7
    assert lib.spider_graph_message_passing_dynamic_f32(p(z), 1, 4, 2, 1, 2, p(eidx), p(z),
                                                        p(asg0), p(z)) == 2
    assert lib.spider_expert_grouped_gemm_f32(p(z), 1, 4, 4, 2, 2, p(asg), p(z), p(z), p(z),
                                              p(z)) == 2  # expert 2 >= E


def test_identity(nat):
    lib = nat.lib()
    assert lib.smoe_abi_version() == 10
    assert lib.smoe_backend_name() == b"hip-gfx950"
    assert lib.smoe_backend_caps() == 0b1111


def _block(nat, **kw):
    b = nat.SmoeBlock()
    b.act_dtype, b.H, b.E, b.K, b.M, b.L, b.R = nat.BF16, 1024, 16, 2, 2, 32, 6
    fake = 0x1000
    b.router_w = b.loop_bias = b.edge_gen_w = b.edge_loop_bias = b.edge_value_w = fake
    ex = b.experts
    ex.format, ex.act, ex.E, ex.H, ex.U = nat.BF16, nat.ACT_SWIGLU, 16, 1024, 2816
    ex.w_up = ex.w_down = fake
    b.alpha, b.beta, b.eps = 0.5, 0.1, 1e-5
    for k, v in kw.items():
        if hasattr(ex, k) and k in ("format", "act", "U", "group_size", "scale_dtype"):
            setattr(ex, k, v)
        else:
            setattr(b, k, v)
    return b


def test_workspace_layout_is_consistent(nat):
    lib = nat.lib()
    b = _block(nat)
    n = 16384
    lay = nat.SmoeWsLayout()
    assert lib.smoe_block_workspace_layout(ctypes.byref(b), n, ctypes.byref(lay)) == 0
    assert lay.total == lib.smoe_block_workspace_bytes(ctypes.byref(b), n)
    offs = sorted((getattr(lay, f), f) for f in nat._LAYOUT_FIELDS if f != "total")
    assert all(o % 256 == 0 for o, _ in offs)
    # the small-step regions are empty at this N (they sit at the end)
    small_only = ("front", "sel_idx", "sel_w", "h_tmp2")
    assert all(getattr(lay, f) == lay.total for f in small_only)
    assert max(o for o, f in offs if f not in small_only) < lay.total
    assert lay.S == 4 and lay.ffn_dtype == nat.BF16
    # E = 16 prefill (the one-pass front): plan scratch for both plans (two
    # [G, C] count matrices each)
    nxt = min(o for o, f in offs if o > lay.scratch)
    assert nxt - lay.scratch >= 2 * 2 * 16 * (n // 64) * 4
    # the per-source edges wait in the edge_logit region in slot order (M <= E / 2)
    assert lay.edge_idx - lay.edge_logit >= n * 2 * 2 * 2 * 4
    # regions do not overlap: each is at least its size from the next
    assert lay.top_idx - lay.logits >= n * 16 * 4
    assert lay.act + n * 2 * 2816 * 2 <= lay.y
    assert lay.proj + n * 4 * 1024 * 2 <= lay.msg
    # a decode-size step (N <= 256, bf16) gets the front region: [N, E + E*E] f32
    small = nat.SmoeWsLayout()
    assert lib.smoe_block_workspace_layout(ctypes.byref(b), 64, ctypes.byref(small)) == 0
    assert small.total - small.front >= 64 * (16 + 16 * 16) * 4
    # and the decode loop's regions: per-token source edges [N, K, M], a second input buffer
    assert small.sel_w - small.sel_idx >= 64 * 2 * 2 * 4
    assert small.h_tmp2 - small.sel_w >= 64 * 2 * 2 * 4
    assert small.total - small.h_tmp2 >= 64 * 1024 * 2


@pytest.mark.parametrize("bad", [dict(K=0), dict(K=17), dict(E=257), dict(E=128, K=16, M=8),
                                 dict(M=0), dict(H=1000),
                                 dict(act_dtype=7), dict(format=9), dict(U=100),
                                 dict(format=3, group_size=48)])
def test_invalid_block_is_rejected_without_launch(nat, bad):
    lib = nat.lib()
    b = _block(nat, **bad)
    if "E" in bad:
        b.experts.E = bad["E"]
    assert lib.smoe_block_workspace_bytes(ctypes.byref(b), 64) == 0
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 0, 1, 0x1000, 1 << 40, None)
    assert rc in (1, -2)
    assert lib.smoe_last_error()


def test_pack_weight_tiles_rejects_bad_shapes(nat):
    lib = nat.lib()
    for g, n, k in [(0, 16, 64), (1, 10, 64), (1, 16, 100), (1, 8, 64)]:
        for code in (nat.BF16, nat.FP8_E4M3):
            assert lib.smoe_pack_weight_tiles(0x1000, code, g, n, k, 0x2000, None) == 1
    assert lib.smoe_pack_weight_tiles(None, nat.BF16, 1, 16, 64, 0x2000, None) == 1
    assert lib.smoe_pack_weight_tiles(0x1008, nat.BF16, 1, 16, 64, 0x2000, None) == 1  # alignment
    for code in (nat.F32, nat.INT4, nat.F16):  # formats without a tile layout
        assert lib.smoe_pack_weight_tiles(0x1000, code, 1, 16, 64, 0x2000, None) == -2


def test_capacity_and_range_errors(nat):
    lib = nat.lib()
    b = _block(nat)
    need = lib.smoe_block_workspace_bytes(ctypes.byref(b), 64)
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 0, 1, 0x1000, need - 1, None)
    assert rc == 3
    rc = lib.smoe_block_forward(ctypes.byref(b), 0x1000, 0x1000, 0x1000, 64, 5, 2, 0x1000, need, None)
    assert rc == 1  # loop range past num_loops
    # N == 0 is a no-op
    assert lib.smoe_block_forward(ctypes.byref(b), None, None, None, 0, 0, 1, None, 0, None) == 0


def test_exit_gate_argument_errors(nat):
    """smoe_block_forward_exit: missing gate buffers, a NaN threshold, a
    short workspace and a bad loop range are rejected before any launch."""
    lib = nat.lib()
    b = _block(nat)
    need = lib.smoe_block_workspace_bytes(ctypes.byref(b), 64)
    p = 0x1000
    f = lambda wb, thr, act, ws_bytes=need, lb=0: lib.smoe_block_forward_exit(
        ctypes.byref(b), p, p, p, 64, lb, 1, wb, thr, act, None, p, ws_bytes, None)
    assert f(None, 0.5, p) == 1
    assert f(p, 0.5, None) == 1
    assert f(p, float("nan"), p) == 1
    assert f(p, 0.5, p, need - 1) == 3
    assert f(p, 0.5, p, need, 6) == 1  # loop 6 of 6


def test_stage_entries_reject_bad_arguments(nat):
    """Shape, dtype, null-buffer and workspace checks of the stage entry
    points run before any launch (no device needed)."""
    lib = nat.lib()
    p = 0x1000  # never dereferenced: every call below fails its checks first
    # edge top-m: E, K, M ranges; ldw; null buffers; workspace size
    assert lib.smoe_edge_topm_workspace_bytes(10, 2, 0, 2) == 0
    assert lib.smoe_edge_topm_workspace_bytes(10, 2, 16, 2) > 0
    args = lambda **o: dict(dict(x=p, adt=nat.BF16, n=10, h=128, w=p, ldw=160, b=p, e=16, k=2, m=2,
                                  src=p, oi=p, ow=p, ws=p, wsb=1 << 30), **o)
    def topm(a):
        return lib.smoe_edge_topm(a["x"], a["adt"], a["n"], a["h"], a["w"], a["ldw"], a["b"],
                                  a["e"], a["k"], a["m"], a["src"], a["oi"], a["ow"], a["ws"],
                                  a["wsb"], None)
    assert topm(args(e=0)) == 1
    assert topm(args(k=17)) == 1
    assert topm(args(m=3, e=2)) == 1
    assert topm(args(h=100)) == 1
    assert topm(args(ldw=100)) == 1
    assert topm(args(ldw=161)) == 1
    assert topm(args(adt=nat.INT4)) == -2
    assert topm(args(src=None)) == 1
    assert topm(args(wsb=16)) == 3
    # edge message
    assert lib.smoe_edge_message_workspace_bytes(10, 128, 16, 2, 2, nat.INT4) == 0
    assert lib.smoe_edge_message_workspace_bytes(10, 128, 16, 2, 2, nat.BF16) > 0
    def msg(**o):
        a = dict(dict(x=p, adt=nat.BF16, n=10, h=128, w=p, t=None, e=16, k=2, m=2, src=p, ei=p,
                      ew=p, out=p, odt=nat.BF16, ws=p, wsb=1 << 30), **o)
        return lib.smoe_edge_message(a["x"], a["adt"], a["n"], a["h"], a["w"], a["t"], a["e"],
                                     a["k"], a["m"], a["src"], a["ei"], a["ew"], a["out"], a["odt"],
                                     a["ws"], a["wsb"], None)
    assert msg(e=257) == 1
    assert msg(odt=nat.INT4) == -2
    assert msg(ei=None) == 1
    assert msg(wsb=16) == 3
    assert msg(n=-1) == 1
    # epilogue
    def epi(**o):
        a = dict(dict(h=p, x0=p, adt=nat.BF16, d=p, ddt=nat.F32, n=10, hid=128), **o)
        return lib.smoe_combine_epilogue(a["h"], a["x0"], a["adt"], a["d"], a["ddt"], a["n"],
                                         a["hid"], 0.5, 0.1, None, None, 1e-5, p, None)
    assert epi(hid=100) == 1
    assert epi(ddt=nat.INT4) == -2
    assert epi(d=None) == 1
    assert epi(adt=nat.FP8_E4M3) == -2
    # N == 0 is a no-op
    assert epi(n=0) == 0
    assert topm(args(n=0)) == 0
    assert msg(n=0) == 0
