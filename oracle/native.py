"""Oracle: the reference's native (torch-free) loop kernels in numpy
(TEST INFRASTRUCTURE ONLY).

Restates the scalar C++ library (kernels/scalar/scalar.cpp:7-104,
scalar_phase1_1.cpp:62-121) and the device ABI that mirrors it
(kernels/cuda/spider_kernels.cu:8-117, spider_expert_v2.cu:13-85), in the
operation order of the scalar code, float32 where it uses float and float64
where it uses double:

  router        p = exp(l + b - max) / sum (sum in index order), k picks of
                the largest p not taken (first index on ties), weights
                p / max(sum of picks, 1e-20)            scalar.cpp:7-34
  graph (v1)    m[b] += (edge_w * route_w) * h[b] per edge of each valid
                source, in slot then CSR order           scalar.cpp:36-53
  experts       act = gelu_tanh(sum_i x_i W_up[e][i][u]) (i ascending);
                out += (route_w act_u) W_down[e][u][:] (u ascending),
                no biases                                scalar.cpp:55-73
  epilogue      u = (h + a d) + b x0 (float); Welford mean / M2 in double;
                inv = 1 / sqrt(float(M2 / H) + eps)       scalar.cpp:75-92
  exit          z = float(sum in double of h_j p_j); conf = the stable
                sigmoid; conf > threshold                scalar.cpp:94-104
  edge project  proj[b,e,j] = float(double sum over i ascending of
                h[b,i] W_edge[e][j][i])              scalar_phase1_1.cpp:17-32
  graph v2      m[b] += edge_w * proj[b, dst] per CSR edge of each valid
                source                                scalar_phase1_1.cpp:34-60
  edge top-m    per (b, src) row: M picks of the first strictly larger
                logit above -inf not yet taken (-1 / -inf when none), then
                exp(w - max) / max(sum in pick order, 1e-20)
                                                      scalar_phase1_2.cpp:11-47
  graph dyn.    m[b] += w[b,src,m] * proj[b, idx[b,src,m]] over the picks
                                                      scalar_phase1_2.cpp:49-72
  edge gen.     logits[b,o] = float(double sum over i of [h; emb]_i
                W_gen[o][i])                          scalar_phase1_3.cpp:14-42
  loop step     logits = h . router_w ([H, E]) in double, router, messages
                (graph v2 over the projection with W_edge and the CSR — the
                host library; graph v1 with the CSR alone — the device ABI's
                loop step; else h), experts, epilogue, exit

Pins (tests/test_oracle_native_forge.py): each function against oracle/_ref
(the reference's scalar library compiled from its sources) — bit for bit
where both run the same float operations, and the reference's own known
answers (kernels/tests/test_kernels.cpp:7-18, 57-59).  The tanh of the
GELU is numpy's (glibc) tanhf in float32; the device's tanhf may differ
by an ulp, so device comparisons of the expert FFN use a tolerance.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def router(logits, bias_row, k):
    """logits [B,E] f32, bias_row [E] -> (w f32 [B,k], idx i32 [B,k])."""
    lg = np.asarray(logits, f32)
    b_, e_ = lg.shape
    bias = np.asarray(bias_row, f32)
    w = np.zeros((b_, k), f32)
    idx = np.zeros((b_, k), np.int32)
    for b in range(b_):
        v = (lg[b] + bias).astype(f32)
        mx = f32(np.max(v))
        s = f32(0)
        for e in range(e_):
            s = f32(s + f32(np.exp(f32(v[e] - mx))))
        p = np.array([f32(f32(np.exp(f32(v[e] - mx))) / s) for e in range(e_)], f32)
        used = np.zeros(e_, bool)
        tot = f32(0)
        for j in range(k):
            best, bv = -1, f32(-1)
            for e in range(e_):
                if not used[e] and p[e] > bv:
                    bv, best = p[e], e
            used[best] = True
            idx[b, j] = best
            w[b, j] = bv
            tot = f32(tot + bv)
        w[b] = (w[b] / f32(max(tot, f32(1e-20)))).astype(f32)
    return w, idx


def graph_v1(h, row_ptr, edge_w, assign, route, nnz=None, loop_idx=0):
    """messages [B,H] of the static CSR graph (scalar.cpp:36-53; sources
    outside [0, E) are skipped, as spider_kernels.cu:28-40 does)."""
    h = np.asarray(h, f32)
    b_, hd = h.shape
    rp = np.asarray(row_ptr)
    e_ = len(rp) - 1
    ew = np.asarray(edge_w, f32).reshape(-1)
    nnz = len(ew) if nnz is None else nnz
    ewl = ew[loop_idx * nnz:(loop_idx + 1) * nnz]
    out = np.zeros((b_, hd), f32)
    for b in range(b_):
        for k in range(assign.shape[1]):
            s = int(assign[b, k])
            if s < 0 or s >= e_:
                continue
            for e in range(int(rp[s]), int(rp[s + 1])):
                if e < nnz:
                    sc = f32(ewl[e] * f32(route[b, k]))
                    out[b] = (out[b] + (sc * h[b]).astype(f32)).astype(f32)
    return out


def gelu_tanh(a):
    a = np.asarray(a, f32)
    c = (f32(0.7978845608) * (a + f32(0.044715) * a * a * a).astype(f32)).astype(f32)
    return (f32(0.5) * a * (f32(1) + np.tanh(c).astype(f32))).astype(f32)


def experts(x, assign, route, w_up, w_down):
    """x [B,H]; w_up [E,H,U]; w_down [E,U,H]; tanh-GELU, no bias."""
    x = np.asarray(x, f32)
    b_, hd = x.shape
    e_ = w_up.shape[0]
    out = np.zeros((b_, hd), f32)
    for b in range(b_):
        for k in range(assign.shape[1]):
            e = int(assign[b, k])
            if e < 0 or e >= e_:
                continue
            a = np.zeros(w_up.shape[2], f32)
            for i in range(hd):
                a = (a + (x[b, i] * w_up[e, i]).astype(f32)).astype(f32)
            act = gelu_tanh(a)
            r = f32(route[b, k])
            for u in range(len(act)):
                out[b] = (out[b] + (f32(r * act[u]) * w_down[e, u]).astype(f32)).astype(f32)
    return out


def epilogue(h, d, x0, alpha, beta, gamma, ln_bias, eps):
    h, d, x0 = (np.asarray(a, f32) for a in (h, d, x0))
    alpha, beta, eps = f32(alpha), f32(beta), f32(eps)
    u = ((h + (alpha * d).astype(f32)).astype(f32) + (beta * x0).astype(f32)).astype(f32)
    out = np.empty_like(u)
    b_, hd = u.shape
    for b in range(b_):
        mean, m2 = 0.0, 0.0
        for j in range(hd):
            v = float(u[b, j])
            dl = v - mean
            mean += dl / (j + 1)
            m2 += dl * (v - mean)
        inv = f32(f32(1) / np.sqrt(f32(f32(m2 / hd) + eps)))
        out[b] = ((((u[b] - f32(mean)).astype(f32) * inv).astype(f32) * gamma).astype(f32)
                  + ln_bias).astype(f32)
    return out


def exit_mask(h, proj, threshold):
    h = np.asarray(h, f32)
    z = (h.astype(np.float64) @ np.asarray(proj, f32).astype(np.float64)).astype(f32)
    conf = np.where(z >= 0, f32(1) / (f32(1) + np.exp(-z)), np.exp(z) / (f32(1) + np.exp(z)))
    return (conf.astype(f32) > f32(threshold)).astype(np.uint8), conf


def _dsum_rows(a, w):
    """out[b, o] = float(double sum over i ascending of a[b, i] w[o, i]):
    every product of two floats is exact in double; the sums are rounded in
    the scalar loop's order."""
    a = np.asarray(a, f32).astype(np.float64)
    w = np.asarray(w, f32).astype(np.float64)
    acc = np.zeros((a.shape[0], w.shape[0]), np.float64)
    for i in range(a.shape[1]):
        acc += a[:, i:i + 1] * w[None, :, i]
    return acc.astype(f32)


def edge_project(h, w_edge):
    """h [B,H], W_edge [E,H,H] -> [B,E,H]."""
    h = np.asarray(h, f32)
    e_, hd, _ = w_edge.shape
    return _dsum_rows(h, np.asarray(w_edge, f32).reshape(e_ * hd, hd)).reshape(-1, e_, hd)


def edge_generator(h, loop_emb, w_gen):
    """[h, loop_emb] . W_gen^T -> [B,E,E] (no bias)."""
    h = np.asarray(h, f32)
    emb = np.asarray(loop_emb, f32).reshape(-1)
    feat = np.concatenate([h, np.broadcast_to(emb, (h.shape[0], emb.size))], axis=1)
    out = _dsum_rows(feat, w_gen)
    e_ = int(round(out.shape[1] ** 0.5))
    return out.reshape(-1, e_, e_)


def edge_topk(logits, m):
    """logits [B,E,E] -> (idx i32 [B,E,M], w f32 [B,E,M])."""
    g = np.asarray(logits, f32)
    b_, e_, _ = g.shape
    idx = np.zeros((b_, e_, m), np.int32)
    w = np.zeros((b_, e_, m), f32)
    for b in range(b_):
        for s in range(e_):
            cand = np.where(np.isnan(g[b, s]), -np.inf, g[b, s]).astype(f32)
            for j in range(m):
                best = int(np.argmax(cand))
                if not cand[best] > -np.inf:
                    idx[b, s, j], w[b, s, j] = -1, -np.inf
                    continue
                idx[b, s, j], w[b, s, j] = best, cand[best]
                cand[best] = -np.inf
            mx = f32(np.max(w[b, s]))
            with np.errstate(invalid="ignore"):  # no pick at all: -inf - -inf
                ex = np.exp((w[b, s] - mx).astype(f32)).astype(f32)
            tot = f32(0)
            for v in ex:
                tot = f32(tot + v)
            w[b, s] = (ex / f32(max(tot, f32(1e-20)))).astype(f32)
    return idx, w


def _graph_proj(proj, assign, edges):
    """m[b] = sum in order of scale * proj[b, dst] over edges(b, src)."""
    proj = np.asarray(proj, f32)
    b_, e_, hd = proj.shape
    out = np.zeros((b_, hd), f32)
    for b in range(b_):
        for k in range(assign.shape[1]):
            s = int(assign[b, k])
            if s < 0 or s >= e_:
                continue
            for dst, sc in edges(b, s):
                if 0 <= dst < e_:
                    out[b] = (out[b] + (f32(sc) * proj[b, dst]).astype(f32)).astype(f32)
    return out


def graph_v2(proj, row_ptr, col_idx, edge_w, assign, nnz=None, loop_idx=0):
    rp = np.asarray(row_ptr)
    ci = np.asarray(col_idx)
    ew = np.asarray(edge_w, f32).reshape(-1)
    nnz = len(ci) if nnz is None else nnz
    ewl = ew[loop_idx * nnz:(loop_idx + 1) * nnz]
    return _graph_proj(proj, assign,
                       lambda b, s: ((int(ci[e]), ewl[e]) for e in range(rp[s], rp[s + 1])))


def graph_dynamic(proj, edge_idx, edge_w, assign):
    ei = np.asarray(edge_idx)
    ew = np.asarray(edge_w, f32)
    return _graph_proj(proj, assign,
                       lambda b, s: ((int(ei[b, s, j]), ew[b, s, j]) for j in range(ei.shape[2])))


def loop_step(h, x0, k, router_w, bias_row, w_up, w_down, gamma, ln_bias, alpha, beta, eps,
              csr=None, exit_proj=None, threshold=0.85, w_edge=None, loop_idx=0):
    """One native loop (scalar_phase1_1.cpp:62-121): returns (h_next, mask,
    assign, route, messages).  csr = (row_ptr, col_idx, edge_w); with
    w_edge the messages are graph v2 over the edge projection (the host
    library, edge weights of loop_idx), without it graph v1 (the device
    ABI's loop step)."""
    h = np.asarray(h, f32)
    logits = _dsum_rows(h, np.asarray(router_w, f32).T)
    route, assign = router(logits, bias_row, k)
    if csr is not None and w_edge is not None:
        msgs = graph_v2(edge_project(h, w_edge), csr[0], csr[1], csr[2], assign,
                        nnz=len(csr[1]), loop_idx=loop_idx)
    elif csr is not None:
        msgs = graph_v1(h, csr[0], csr[2], assign, route, nnz=len(csr[1]))
    else:
        msgs = h.copy()
    delta = experts(msgs, assign, route, w_up, w_down)
    h_next = epilogue(h, delta, x0, alpha, beta, gamma, ln_bias, eps)
    mask = exit_mask(h_next, exit_proj, threshold)[0] if exit_proj is not None else \
        np.zeros(h.shape[0], np.uint8)
    return h_next, mask, assign, route, msgs
