"""ctypes binding of the reference's scalar C++ library (TEST INFRASTRUCTURE).

``oracle/Makefile`` compiles the reference's own scalar sources
(kernels/scalar/scalar*.cpp, kernels/src/{dispatch,phase1_api_ext}.cpp) into
``oracle/_ref/libspider_ref.so``.  The entry points bound here follow
kernels/include/spider_kernels.h:26-121.  They are used only to check the
oracle; ``available()`` is False where the library was not built (the GPU box
builds nothing from the reference, which is absent there).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB = None
_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_ref", "libspider_ref.so")

_f32p = ctypes.POINTER(ctypes.c_float)
_i32p = ctypes.POINTER(ctypes.c_int32)


def available() -> bool:
    return os.path.exists(_PATH)


def lib():
    global _LIB
    if _LIB is None:
        _LIB = ctypes.CDLL(_PATH)
    return _LIB


def _fp(a):
    return a.ctypes.data_as(_f32p)


def _ip(a):
    return a.ctypes.data_as(_i32p)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def router_f32(logits, loop_bias, k, loop_idx):
    """spider_router_f32 (scalar.cpp:7-34): logits [B,E], loop_bias [R,E]."""
    logits = _f32(logits)
    bias = _f32(loop_bias)
    b, e = logits.shape
    w = np.zeros((b, k), np.float32)
    i = np.zeros((b, k), np.int32)
    rc = lib().spider_router_f32(_fp(logits), _fp(bias), b, e, k, loop_idx, _fp(w), _ip(i))
    return rc, w, i


def edge_topk_f32(edge_logits, m):
    """spider_edge_topk_f32 (scalar_phase1_2.cpp:11-47): logits [B,E,E]."""
    g = _f32(edge_logits)
    b, e, _ = g.shape
    idx = np.zeros((b, e, m), np.int32)
    w = np.zeros((b, e, m), np.float32)
    rc = lib().spider_edge_topk_f32(_fp(g), b, e, m, _ip(idx), _fp(w))
    return rc, idx, w


def edge_generator_f32(hidden, loop_emb_row, w_gen):
    """spider_edge_generator_f32 (scalar_phase1_3.cpp:14-42), no bias."""
    h = _f32(hidden)
    emb = _f32(loop_emb_row)
    wg = _f32(w_gen)
    b, hid = h.shape
    e2 = wg.shape[0]
    e = int(round(e2 ** 0.5))
    out = np.zeros((b, e2), np.float32)
    rc = lib().spider_edge_generator_f32(_fp(h), b, hid, e, _fp(emb), emb.size, _fp(wg), _fp(out))
    return rc, out.reshape(b, e, e)


def graph_dynamic_with_edge_value_f32(hidden, w_edge, edge_idx, edge_w, assign):
    """spider_graph_dynamic_with_edge_value_f32 (scalar_phase1_2.cpp:74-86)."""
    h = _f32(hidden)
    we = _f32(w_edge)
    ei = np.ascontiguousarray(edge_idx, np.int32)
    ew = _f32(edge_w)
    asg = np.ascontiguousarray(assign, np.int32)
    b, hid = h.shape
    e = we.shape[0]
    k = asg.shape[1]
    m = ei.shape[2]
    msg = np.zeros((b, hid), np.float32)
    tmp = np.zeros((b, e, hid), np.float32)
    rc = lib().spider_graph_dynamic_with_edge_value_f32(
        _fp(h), b, hid, e, k, m, _fp(we), _ip(ei), _fp(ew), _ip(asg), _fp(msg), _fp(tmp))
    return rc, msg


def expert_grouped_gemm_f32(tokens, assign, route, w_up_ehu, w_down_euh):
    """spider_expert_grouped_gemm_f32 (scalar.cpp:55-73): tanh-GELU, no bias,
    W_up [E,H,U], W_down [E,U,H]."""
    x = _f32(tokens)
    asg = np.ascontiguousarray(assign, np.int32)
    rw = _f32(route)
    wu = _f32(w_up_ehu)
    wd = _f32(w_down_euh)
    b, hid = x.shape
    e, _, u = wu.shape
    k = asg.shape[1]
    out = np.zeros((b, hid), np.float32)
    rc = lib().spider_expert_grouped_gemm_f32(
        _fp(x), b, hid, u, e, k, _ip(asg), _fp(rw), _fp(wu), _fp(wd), _fp(out))
    return rc, out


def loop_epilogue_f32(h, delta, x0, alpha, beta, ln_w, ln_b, eps):
    """spider_loop_epilogue_f32 (scalar.cpp:75-92)."""
    h = _f32(h)
    d = _f32(delta)
    x = _f32(x0)
    g = _f32(ln_w)
    lb = _f32(ln_b)
    b, hid = h.shape
    out = np.zeros_like(h)
    lib().spider_loop_epilogue_f32.argtypes = [
        _f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_float,
        _f32p, _f32p, ctypes.c_float, _f32p]
    rc = lib().spider_loop_epilogue_f32(_fp(h), _fp(d), _fp(x), b, hid, alpha, beta,
                                        _fp(g), _fp(lb), eps, _fp(out))
    return rc, out


def graph_message_passing_f32(hidden, row_ptr, col_idx, edge_w, assign, route, loop_idx=0):
    """spider_graph_message_passing_f32 (scalar.cpp:36-53): the static CSR
    graph with route weights (v1)."""
    h = _f32(hidden)
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_idx, np.int32)
    ew = _f32(edge_w)
    asg = np.ascontiguousarray(assign, np.int32)
    rw = _f32(route)
    b, hid = h.shape
    e = len(rp) - 1
    out = np.zeros_like(h)
    rc = lib().spider_graph_message_passing_f32(_fp(h), b, hid, e, asg.shape[1], _ip(rp), _ip(ci),
                                                _fp(ew), len(ci), loop_idx, _ip(asg), _fp(rw),
                                                _fp(out))
    return rc, out


def early_exit_f32(h, proj, threshold):
    """spider_early_exit_f32 (scalar.cpp:94-104)."""
    h = _f32(h)
    p = _f32(proj)
    b, hid = h.shape
    mask = np.zeros(b, np.uint8)
    lib().spider_early_exit_f32.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int,
                                            ctypes.c_float, ctypes.POINTER(ctypes.c_uint8)]
    rc = lib().spider_early_exit_f32(_fp(h), _fp(p), b, hid, threshold,
                                     mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return rc, mask


def edge_project_f32(hidden, w_edge):
    """spider_edge_project_f32 (scalar_phase1_1.cpp:17-32): W_edge [E,H,H]."""
    h = _f32(hidden)
    we = _f32(w_edge)
    b, hid = h.shape
    e = we.shape[0]
    out = np.zeros((b, e, hid), np.float32)
    rc = lib().spider_edge_project_f32(_fp(h), b, hid, e, _fp(we), _fp(out))
    return rc, out


def graph_v2_f32(projected, row_ptr, col_idx, edge_w, assign, loop_idx=0):
    """spider_graph_message_passing_v2_f32 (scalar_phase1_1.cpp:34-60)."""
    p = _f32(projected)
    rp = np.ascontiguousarray(row_ptr, np.int32)
    ci = np.ascontiguousarray(col_idx, np.int32)
    ew = _f32(edge_w)
    asg = np.ascontiguousarray(assign, np.int32)
    b, e, hid = p.shape
    out = np.zeros((b, hid), np.float32)
    rc = lib().spider_graph_message_passing_v2_f32(_fp(p), b, hid, e, asg.shape[1], _ip(rp),
                                                   _ip(ci), _fp(ew), len(ci), loop_idx, _ip(asg),
                                                   _fp(out))
    return rc, out


def graph_dynamic_f32(projected, edge_idx, edge_w, assign):
    """spider_graph_message_passing_dynamic_f32 (scalar_phase1_2.cpp:49-72)."""
    p = _f32(projected)
    ei = np.ascontiguousarray(edge_idx, np.int32)
    ew = _f32(edge_w)
    asg = np.ascontiguousarray(assign, np.int32)
    b, e, hid = p.shape
    out = np.zeros((b, hid), np.float32)
    rc = lib().spider_graph_message_passing_dynamic_f32(_fp(p), b, hid, e, asg.shape[1],
                                                        ei.shape[2], _ip(ei), _fp(ew), _ip(asg),
                                                        _fp(out))
    return rc, out


def moe_loop_step_f32(h, x0, k, loop_idx, router_w, loop_bias, w_up, w_down, ln_w, ln_b, alpha,
                      beta, eps, exit_proj=None, threshold=0.85, csr=None, w_edge=None):
    """spider_moe_loop_step_f32 (scalar_phase1_1.cpp:62-121); csr =
    (row_ptr, col_idx, edge_w [R*nnz]) with w_edge [E,H,H] selects the
    edge-value graph, otherwise messages = h."""
    h = _f32(h)
    x = _f32(x0)
    rw = _f32(router_w)
    lb = _f32(loop_bias)
    wu = _f32(w_up)
    wd = _f32(w_down)
    g = _f32(ln_w)
    gb = _f32(ln_b)
    b, hid = h.shape
    e = rw.shape[1]
    u = wu.shape[2]
    out = np.zeros_like(h)
    mask = np.zeros(b, np.uint8)
    asg = np.zeros((b, k), np.int32)
    route = np.zeros((b, k), np.float32)
    msgs = np.zeros_like(h)
    ep = None if exit_proj is None else _f32(exit_proj)
    c_i, c_f, vp = ctypes.c_int, ctypes.c_float, ctypes.c_void_p
    fn = lib().spider_moe_loop_step_f32
    fn.argtypes = [vp, vp, c_i, c_i, c_i, c_i, c_i, c_i, vp, vp, vp, vp, vp, c_i, vp, vp, vp,
                   vp, vp, c_f, c_f, c_f, vp, c_f, vp, vp, vp, vp, vp]
    ptr = lambda a: None if a is None else a.ctypes.data  # noqa: E731
    rp = ci = ew = we = None
    nnz = 0
    if csr is not None:
        rp = np.ascontiguousarray(csr[0], np.int32)
        ci = np.ascontiguousarray(csr[1], np.int32)
        ew = _f32(csr[2])
        nnz = len(ci)
    if w_edge is not None:
        we = _f32(w_edge)
    rc = fn(ptr(h), ptr(x), b, hid, e, k, u, loop_idx, ptr(rw), ptr(lb), ptr(rp), ptr(ci),
            ptr(ew), nnz, ptr(we), ptr(wu), ptr(wd), ptr(g), ptr(gb), alpha, beta, eps, ptr(ep),
            threshold, ptr(out), ptr(mask), ptr(asg), ptr(route), ptr(msgs))
    return rc, out, mask, asg, route
