"""The reference's native loop on the GPU: the device ABI of
include/spider_cuda.h (spider_cuda_* in libsmoe.so) behind the method names
of the reference's numpy binding (kernels/python/spider_native.py:196-480,
NativeKernels) and the torch-free loop step of
spider_infer/orbit/native_backend.py:309-388.

HipKernels takes numpy arrays or torch tensors; numpy inputs are copied to
the GPU and results come back as numpy (the binding's contract), torch
tensors stay on the GPU.  Argument errors raise RuntimeError("<fn> failed:
rc") like the reference's wrappers (spider_native.py:224-225).

NativeLoop runs loops of the block from a .spiderw bundle (spiderw.py) with
spider_cuda_moe_loop_step_f32: the reference's fp32 native semantics (router
on h . router_w, static CSR message pass with route weights, tanh-GELU
experts without biases, LayerNorm, exit mask) — not the PyTorch block's.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _native as nat
from .spiderw import SpiderWBundle, load_spiderw


def _rc(rc: int, fn: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{fn} failed: {rc}")


class HipKernels:
    """spider_native.NativeKernels' router / graph / expert_ffn / epilogue /
    early_exit, computed by the spider_cuda_* kernels."""

    def __init__(self, device: str | torch.device = "cuda"):
        self.device = torch.device(device)
        self.lib = nat.lib()

    @property
    def backend(self) -> str:
        return "hip-gfx950"

    @property
    def has_cuda(self) -> bool:
        return True

    # ---------------------------------------------------------- plumbing ----
    def _dev(self, a, dtype):
        if isinstance(a, torch.Tensor):
            return a.to(device=self.device, dtype=dtype).contiguous()
        return torch.from_numpy(np.ascontiguousarray(a)).to(device=self.device, dtype=dtype)

    @staticmethod
    def _back(t: torch.Tensor, like):
        if isinstance(like, torch.Tensor):
            return t
        torch.cuda.synchronize(t.device)
        return t.cpu().numpy()

    def _stream(self) -> int:
        return nat.stream_of(self.device)

    # ----------------------------------------------------------- kernels ----
    def router(self, logits, loop_bias, k: int, loop_idx: int = 0):
        """logits [B,E], loop_bias [R,E] (or [E] with loop_idx 0) ->
        (weights f32 [B,k], indices i32 [B,k])."""
        lg = self._dev(logits, torch.float32)
        bias = self._dev(loop_bias, torch.float32)
        b, e = lg.shape
        w = torch.empty(b, k, dtype=torch.float32, device=self.device)
        idx = torch.empty(b, k, dtype=torch.int32, device=self.device)
        _rc(self.lib.spider_cuda_router_f32(lg.data_ptr(), bias.data_ptr(), b, e, k, loop_idx,
                                            w.data_ptr(), idx.data_ptr(), self._stream()),
            "spider_cuda_router_f32")
        return self._back(w, logits), self._back(idx, logits)

    def graph(self, hidden, row_ptr, col_idx, edge_w, assign, route, E: int, loop_idx: int = 0):
        """Static CSR message pass with route weights (v1)."""
        h = self._dev(hidden, torch.float32)
        rp = self._dev(row_ptr, torch.int32)
        ci = self._dev(col_idx, torch.int32)
        ew = self._dev(edge_w, torch.float32)
        asg = self._dev(assign, torch.int32)
        rw = self._dev(route, torch.float32)
        b, hd = h.shape
        out = torch.empty_like(h)
        _rc(self.lib.spider_cuda_graph_message_passing_f32(
            h.data_ptr(), b, hd, E, asg.shape[1], rp.data_ptr(), ci.data_ptr(), ew.data_ptr(),
            int(ci.shape[0]), loop_idx, asg.data_ptr(), rw.data_ptr(), out.data_ptr(),
            self._stream()), "spider_cuda_graph_message_passing_f32")
        return self._back(out, hidden)

    def expert_ffn(self, tokens, assign, route, W_up, W_down, E: int, workspace: bool = False):
        """tanh-GELU experts without biases; W_up [E,H,U], W_down [E,U,H].
        workspace: the v2 entry (hidden activations in a [B,K,U] buffer)."""
        x = self._dev(tokens, torch.float32)
        asg = self._dev(assign, torch.int32)
        rw = self._dev(route, torch.float32)
        wu = self._dev(W_up, torch.float32)
        wd = self._dev(W_down, torch.float32)
        b, h = x.shape
        u, k = wu.shape[-1], asg.shape[1]
        out = torch.empty_like(x)
        if workspace:
            ws = torch.empty(self.lib.spider_cuda_expert_workspace_bytes(b, k, u) // 4,
                             dtype=torch.float32, device=self.device)
            _rc(self.lib.spider_cuda_expert_grouped_gemm_v2_f32(
                x.data_ptr(), b, h, u, E, k, asg.data_ptr(), rw.data_ptr(), wu.data_ptr(),
                wd.data_ptr(), out.data_ptr(), ws.data_ptr(), self._stream()),
                "spider_cuda_expert_grouped_gemm_v2_f32")
        else:
            _rc(self.lib.spider_cuda_expert_grouped_gemm_f32(
                x.data_ptr(), b, h, u, E, k, asg.data_ptr(), rw.data_ptr(), wu.data_ptr(),
                wd.data_ptr(), out.data_ptr(), self._stream()),
                "spider_cuda_expert_grouped_gemm_f32")
        return self._back(out, tokens)

    def epilogue(self, h, delta, x0, gamma, bias, alpha: float = 1.0, beta: float = 0.0,
                 eps: float = 1e-5):
        hh = self._dev(h, torch.float32)
        d = self._dev(delta, torch.float32)
        x = self._dev(x0, torch.float32)
        g = self._dev(gamma, torch.float32)
        lb = self._dev(bias, torch.float32)
        b, hd = hh.shape
        out = torch.empty_like(hh)
        _rc(self.lib.spider_cuda_loop_epilogue_f32(hh.data_ptr(), d.data_ptr(), x.data_ptr(), b,
                                                   hd, float(alpha), float(beta), g.data_ptr(),
                                                   lb.data_ptr(), float(eps), out.data_ptr(),
                                                   self._stream()),
            "spider_cuda_loop_epilogue_f32")
        return self._back(out, h)

    def early_exit(self, h, proj, threshold: float = 0.85):
        hh = self._dev(h, torch.float32)
        p = self._dev(proj, torch.float32).reshape(-1)
        b, hd = hh.shape
        mask = torch.empty(b, dtype=torch.uint8, device=self.device)
        _rc(self.lib.spider_cuda_early_exit_f32(hh.data_ptr(), p.data_ptr(), b, hd,
                                                float(threshold), mask.data_ptr(),
                                                self._stream()),
            "spider_cuda_early_exit_f32")
        return self._back(mask, h)

    def moe_loop_step(self, h, x0, loop_idx: int, *, router_w, loop_bias, W_up, W_down,
                      ln_weight, ln_bias, top_k: int, alpha: float, beta: float,
                      eps: float = 1e-5, csr=None, exit_proj=None, exit_threshold: float = 0.85):
        """spider_cuda_moe_loop_step_f32: (h_next [B,H], exit_mask u8 [B],
        assign [B,K], route [B,K]).  router_w [H,E]; csr = (row_ptr,
        col_idx, edge_w [R?, nnz]) or None (messages = h)."""
        hh = self._dev(h, torch.float32)
        x = self._dev(x0, torch.float32)
        rw = self._dev(router_w, torch.float32)
        lb = self._dev(loop_bias, torch.float32)
        wu = self._dev(W_up, torch.float32)
        wd = self._dev(W_down, torch.float32)
        g = self._dev(ln_weight, torch.float32)
        gb = self._dev(ln_bias, torch.float32)
        b, hd = hh.shape
        e = rw.shape[1]
        u = wu.shape[-1]
        rp = ci = ew = None
        nnz = 0
        if csr is not None:
            rp, ci, ew = (self._dev(csr[0], torch.int32), self._dev(csr[1], torch.int32),
                          self._dev(csr[2], torch.float32))
            nnz = int(ci.shape[0])
        ep = None if exit_proj is None else self._dev(exit_proj, torch.float32).reshape(-1)
        h_next = torch.empty_like(hh)
        mask = torch.empty(b, dtype=torch.uint8, device=self.device)
        assign = torch.empty(b, top_k, dtype=torch.int32, device=self.device)
        route = torch.empty(b, top_k, dtype=torch.float32, device=self.device)
        msgs = torch.empty_like(hh)
        _rc(self.lib.spider_cuda_moe_loop_step_f32(
            hh.data_ptr(), x.data_ptr(), b, hd, e, top_k, u, loop_idx, rw.data_ptr(),
            lb.data_ptr(), nat.ptr(rp), nat.ptr(ci), nat.ptr(ew), nnz, wu.data_ptr(),
            wd.data_ptr(), g.data_ptr(), gb.data_ptr(), float(alpha), float(beta), float(eps),
            nat.ptr(ep), float(exit_threshold), h_next.data_ptr(), mask.data_ptr(),
            assign.data_ptr(), route.data_ptr(), msgs.data_ptr(), self._stream()),
            "spider_cuda_moe_loop_step_f32")
        return (self._back(h_next, h), self._back(mask, h), self._back(assign, h),
                self._back(route, h))


    # ------------------------------------------- dynamic-edge functions ----
    def edge_project(self, hidden, W_edge):
        """[B,E,H] = hidden . W_edge[e]^T per expert (double sums)."""
        h = self._dev(hidden, torch.float32)
        w = self._dev(W_edge, torch.float32)
        b, hd = h.shape
        e = w.shape[0]
        out = torch.empty(b, e, hd, dtype=torch.float32, device=self.device)
        _rc(self.lib.spider_cuda_edge_project_f32(h.data_ptr(), b, hd, e, w.data_ptr(),
                                                  out.data_ptr(), self._stream()),
            "spider_cuda_edge_project_f32")
        return self._back(out, hidden)

    def graph_v2(self, projected, row_ptr, col_idx, edge_w, assign, E: int, loop_idx: int = 0):
        p = self._dev(projected, torch.float32)
        rp = self._dev(row_ptr, torch.int32)
        ci = self._dev(col_idx, torch.int32)
        ew = self._dev(edge_w, torch.float32)
        asg = self._dev(assign, torch.int32)
        b, _, hd = p.shape
        out = torch.empty(b, hd, dtype=torch.float32, device=self.device)
        _rc(self.lib.spider_cuda_graph_message_passing_v2_f32(
            p.data_ptr(), b, hd, E, asg.shape[1], rp.data_ptr(), ci.data_ptr(), ew.data_ptr(),
            int(ci.shape[0]), loop_idx, asg.data_ptr(), out.data_ptr(), self._stream()),
            "spider_cuda_graph_message_passing_v2_f32")
        return self._back(out, projected)

    def edge_topk(self, edge_logits, M: int):
        g = self._dev(edge_logits, torch.float32)
        if g.ndim == 2:
            g = g.unsqueeze(0)
        b, e, _ = g.shape
        idx = torch.empty(b, e, M, dtype=torch.int32, device=self.device)
        w = torch.empty(b, e, M, dtype=torch.float32, device=self.device)
        _rc(self.lib.spider_cuda_edge_topk_f32(g.data_ptr(), b, e, M, idx.data_ptr(), w.data_ptr(),
                                               self._stream()), "spider_cuda_edge_topk_f32")
        return self._back(idx, edge_logits), self._back(w, edge_logits)

    def edge_generator(self, hidden, loop_emb, W_gen, E: int):
        h = self._dev(hidden, torch.float32)
        emb = self._dev(loop_emb, torch.float32).reshape(-1)
        w = self._dev(W_gen, torch.float32)
        b, hd = h.shape
        out = torch.empty(b, E, E, dtype=torch.float32, device=self.device)
        _rc(self.lib.spider_cuda_edge_generator_f32(h.data_ptr(), b, hd, E, emb.data_ptr(),
                                                    int(emb.numel()), w.data_ptr(),
                                                    out.data_ptr(), self._stream()),
            "spider_cuda_edge_generator_f32")
        return self._back(out, hidden)

    def graph_dynamic(self, projected, edge_indices, edge_weights, assign, E: int, M: int):
        p = self._dev(projected, torch.float32)
        ei = self._dev(edge_indices, torch.int32)
        ew = self._dev(edge_weights, torch.float32)
        asg = self._dev(assign, torch.int32)
        b, _, hd = p.shape
        out = torch.empty(b, hd, dtype=torch.float32, device=self.device)
        _rc(self.lib.spider_cuda_graph_message_passing_dynamic_f32(
            p.data_ptr(), b, hd, E, asg.shape[1], M, ei.data_ptr(), ew.data_ptr(), asg.data_ptr(),
            out.data_ptr(), self._stream()), "spider_cuda_graph_message_passing_dynamic_f32")
        return self._back(out, projected)

    def graph_from_generator(self, hidden, loop_emb, W_gen, W_edge, assign, E: int, M: int):
        logits = self.edge_generator(hidden, loop_emb, W_gen, E)
        edge_idx, edge_w = self.edge_topk(logits, M)
        projected = self.edge_project(hidden, W_edge)
        return self.graph_dynamic(projected, edge_idx, edge_w, assign, E, M)


def _host_f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _host_i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


class HostKernels:
    """The reference's numpy binding (kernels/python/spider_native.py:196-480,
    NativeKernels) over the host entry points of include/spider_kernels.h:
    numpy arrays in and out, the compute on the GPU (libsmoe.so copies the
    inputs to the current device and the results back).  Errors raise
    RuntimeError("<fn> failed: rc") as there."""

    def __init__(self):
        self.lib = nat.lib()

    @property
    def backend(self) -> str:
        return self.lib.spider_backend_name().decode()

    @property
    def caps(self) -> int:
        return int(self.lib.spider_backend_caps())

    @property
    def has_cuda(self) -> bool:
        return True

    def _call(self, name: str, *args):
        rc = getattr(self.lib, name)(*[a.ctypes.data if isinstance(a, np.ndarray) else a
                                       for a in args])
        if rc != 0:
            raise RuntimeError(f"{name} failed: {rc}")

    def router(self, logits, loop_bias, k: int, loop_idx: int = 0):
        lg, bias = _host_f32(logits), _host_f32(loop_bias)
        b, e = lg.shape
        w = np.zeros((b, k), np.float32)
        idx = np.zeros((b, k), np.int32)
        self._call("spider_router_f32", lg, bias, b, e, k, loop_idx, w, idx)
        return w, idx

    def graph(self, hidden, row_ptr, col_idx, edge_w, assign, route, E: int, loop_idx: int = 0):
        h = _host_f32(hidden)
        b, hd = h.shape
        asg = _host_i32(assign)
        ci = _host_i32(col_idx)
        out = np.zeros_like(h)
        self._call("spider_graph_message_passing_f32", h, b, hd, E, asg.shape[1],
                   _host_i32(row_ptr), ci, _host_f32(edge_w), int(ci.shape[0]), loop_idx, asg,
                   _host_f32(route), out)
        return out

    def edge_project(self, hidden, W_edge):
        h, w = _host_f32(hidden), _host_f32(W_edge)
        b, hd = h.shape
        out = np.zeros((b, w.shape[0], hd), np.float32)
        self._call("spider_edge_project_f32", h, b, hd, w.shape[0], w, out)
        return out

    def graph_v2(self, projected, row_ptr, col_idx, edge_w, assign, E: int, loop_idx: int = 0):
        p = _host_f32(projected)
        b, _, hd = p.shape
        asg = _host_i32(assign)
        ci = _host_i32(col_idx)
        out = np.zeros((b, hd), np.float32)
        self._call("spider_graph_message_passing_v2_f32", p, b, hd, E, asg.shape[1],
                   _host_i32(row_ptr), ci, _host_f32(edge_w), int(ci.shape[0]), loop_idx, asg,
                   out)
        return out

    def edge_topk(self, edge_logits, M: int):
        g = _host_f32(edge_logits)
        if g.ndim == 2:
            g = g.reshape(1, *g.shape)
        b, e, _ = g.shape
        idx = np.zeros((b, e, M), np.int32)
        w = np.zeros((b, e, M), np.float32)
        self._call("spider_edge_topk_f32", g, b, e, M, idx, w)
        return idx, w

    def edge_generator(self, hidden, loop_emb, W_gen, E: int):
        h = _host_f32(hidden)
        emb = _host_f32(loop_emb).reshape(-1)
        b, hd = h.shape
        out = np.zeros((b, E * E), np.float32)
        self._call("spider_edge_generator_f32", h, b, hd, E, emb, int(emb.shape[0]),
                   _host_f32(W_gen), out)
        return out.reshape(b, E, E)

    def graph_dynamic(self, projected, edge_indices, edge_weights, assign, E: int, M: int):
        p = _host_f32(projected)
        b, _, hd = p.shape
        asg = _host_i32(assign)
        out = np.zeros((b, hd), np.float32)
        self._call("spider_graph_message_passing_dynamic_f32", p, b, hd, E, asg.shape[1], M,
                   _host_i32(edge_indices), _host_f32(edge_weights), asg, out)
        return out

    def graph_from_generator(self, hidden, loop_emb, W_gen, W_edge, assign, E: int, M: int):
        """spider_graph_from_generator_f32 in one call (the reference's
        binding composes the four steps; the result is the same)."""
        h = _host_f32(hidden)
        emb = _host_f32(loop_emb).reshape(-1)
        b, hd = h.shape
        asg = _host_i32(assign)
        msg = np.zeros((b, hd), np.float32)
        logits = np.zeros((b, E * E), np.float32)
        eidx = np.zeros((b, E, M), np.int32)
        ew = np.zeros((b, E, M), np.float32)
        proj = np.zeros((b, E, hd), np.float32)
        self._call("spider_graph_from_generator_f32", h, b, hd, E, asg.shape[1], M, emb,
                   int(emb.shape[0]), _host_f32(W_gen), _host_f32(W_edge), asg, msg, logits,
                   eidx, ew, proj)
        return msg

    def expert_ffn(self, tokens, assign, route, W_up, W_down, E: int):
        x = _host_f32(tokens)
        b, hd = x.shape
        wu = _host_f32(W_up)
        asg = _host_i32(assign)
        out = np.zeros_like(x)
        self._call("spider_expert_grouped_gemm_f32", x, b, hd, wu.shape[-1], E, asg.shape[1], asg,
                   _host_f32(route), wu, _host_f32(W_down), out)
        return out

    def epilogue(self, h, delta, x0, gamma, bias, alpha: float = 1.0, beta: float = 0.0,
                 eps: float = 1e-5):
        hh = _host_f32(h)
        b, hd = hh.shape
        out = np.zeros_like(hh)
        self._call("spider_loop_epilogue_f32", hh, _host_f32(delta), _host_f32(x0), b, hd,
                   float(alpha), float(beta), _host_f32(gamma), _host_f32(bias), float(eps), out)
        return out

    def early_exit(self, h, proj, threshold: float = 0.85):
        hh = _host_f32(h)
        b, hd = hh.shape
        mask = np.zeros(b, np.uint8)
        self._call("spider_early_exit_f32", hh, _host_f32(proj).reshape(-1), b, hd,
                   float(threshold), mask)
        return mask

    def moe_loop_step(self, h, x0, loop_idx: int, *, router_w, loop_bias, W_up, W_down,
                      ln_weight, ln_bias, top_k: int, alpha: float, beta: float,
                      eps: float = 1e-5, csr=None, W_edge=None, exit_proj=None,
                      exit_threshold: float = 0.85):
        """spider_moe_loop_step_f32: (h_next, exit_mask, assign, route,
        messages); the projected CSR pass when both csr = (row_ptr, col_idx,
        edge_w [R*nnz]) and W_edge [E,H,H] are given, else messages = h."""
        hh = _host_f32(h)
        b, hd = hh.shape
        rw = _host_f32(router_w)
        e = rw.shape[1]
        wu = _host_f32(W_up)
        out = np.zeros_like(hh)
        mask = np.zeros(b, np.uint8)
        asg = np.zeros((b, top_k), np.int32)
        route = np.zeros((b, top_k), np.float32)
        msgs = np.zeros_like(hh)
        rp = ci = ew = None
        nnz = 0
        if csr is not None:
            rp, ci, ew = _host_i32(csr[0]), _host_i32(csr[1]), _host_f32(csr[2])
            nnz = int(ci.shape[0])
        we = None if W_edge is None else _host_f32(W_edge)
        ep = None if exit_proj is None else _host_f32(exit_proj).reshape(-1)
        self._call("spider_moe_loop_step_f32", hh, _host_f32(x0), b, hd, e, top_k, wu.shape[-1],
                   loop_idx, rw, _host_f32(loop_bias), rp, ci, ew, nnz, we, wu, _host_f32(W_down),
                   _host_f32(ln_weight), _host_f32(ln_bias), float(alpha), float(beta),
                   float(eps), ep, float(exit_threshold), out, mask, asg, route, msgs)
        return out, mask, asg, route, msgs


class NativeLoop:
    """The block loops of a .spiderw bundle on the GPU (the loop body of
    native_backend.py:309-388 with the device ABI's static graph)."""

    def __init__(self, bundle: SpiderWBundle | str, *, residual_scale: float = 0.5,
                 reinject_weight: float = 0.1, eps: float = 1e-5, early_exit: bool = False,
                 exit_threshold: float = 0.85, device="cuda"):
        self.bundle = load_spiderw(bundle) if isinstance(bundle, str) else bundle
        self.kernels = HipKernels(device)
        self.alpha, self.beta, self.eps = residual_scale, reinject_weight, eps
        self.early_exit, self.exit_threshold = early_exit, exit_threshold
        m = self.bundle.meta
        dev = self.kernels.device
        t = self.bundle.tensors
        h = m.hidden_size
        router = np.asarray(t["router"], dtype=np.float32)
        self.router_w = torch.from_numpy(router if router.shape[0] == h else router.T.copy()).to(dev)
        lb = np.asarray(t["loop_bias"], dtype=np.float32)
        self.loop_bias = torch.from_numpy(lb.reshape(-1, m.num_experts)).to(dev)
        self.w_up = torch.from_numpy(np.asarray(t["expert_up"], dtype=np.float32)).to(dev)
        self.w_down = torch.from_numpy(np.asarray(t["expert_down"], dtype=np.float32)).to(dev)
        norm = np.asarray(t["moe_norm"], dtype=np.float32)
        gamma, beta = (norm, np.zeros_like(norm)) if norm.ndim == 1 else (norm[0], norm[1])
        self.gamma = torch.from_numpy(gamma.copy()).to(dev)
        self.ln_bias = torch.from_numpy(beta.copy()).to(dev)
        self.csr = None
        if self.bundle.csr is not None and self.bundle.csr.get("row_ptr") is not None:
            c = self.bundle.csr
            self.csr = tuple(torch.from_numpy(np.ascontiguousarray(c[k])).to(dev)
                             for k in ("row_ptr", "col_idx", "edge_w"))
        ex = t.get("exit_head")
        self.exit_proj = None if ex is None else torch.from_numpy(
            np.asarray(ex, dtype=np.float32).reshape(-1).copy()).to(dev)

    def moe_loop_step(self, h, x0, loop_idx: int):
        m = self.bundle.meta
        bias_row = min(loop_idx, self.loop_bias.shape[0] - 1)
        graph_loop = min(loop_idx, max(m.num_loops - 1, 0))
        csr = self.csr
        if csr is not None:
            nnz = csr[1].shape[0]
            ew = csr[2].reshape(-1)
            if ew.numel() >= nnz * (graph_loop + 1):
                csr = (csr[0], csr[1], ew[graph_loop * nnz:(graph_loop + 1) * nnz])
            else:
                csr = (csr[0], csr[1], ew[:nnz])
        h_next, mask, _, _ = self.kernels.moe_loop_step(
            h, x0, 0, router_w=self.router_w, loop_bias=self.loop_bias[bias_row:bias_row + 1],
            W_up=self.w_up, W_down=self.w_down, ln_weight=self.gamma, ln_bias=self.ln_bias,
            top_k=m.top_k, alpha=self.alpha, beta=self.beta, eps=self.eps, csr=csr,
            exit_proj=self.exit_proj if self.early_exit else None,
            exit_threshold=self.exit_threshold)
        return h_next, mask

    def run_loops(self, h, max_loops: int | None = None):
        x0 = h
        n = self.bundle.meta.num_loops if max_loops is None else max_loops
        for r in range(n):
            h, _ = self.moe_loop_step(h, x0, r)
        return h


__all__ = ["HipKernels", "HostKernels", "NativeLoop"]
