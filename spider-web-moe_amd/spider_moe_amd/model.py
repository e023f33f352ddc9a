"""SpiderMoELayer / SpiderWebLM with the reference's call surface, running the
block on gfx950 HIP kernels (libsmoe.so).

SpiderMoELayer mirrors spider_moe/model.py:163-349: the same constructor,
parameter names and shapes (so ``state_dict`` keys load either way),
``forward(h, x0, loop_idx, return_stats=False)``, ``quantize_experts`` /
``dequantize_experts``.  The forward is one native call
(``smoe_block_forward``): router, edge graph, both dispatch plans, grouped
GEMMs and the LayerNorm epilogue run as HIP kernels on the current stream.
The parameters are packed once into the kernels' stacked layout and re-packed
only when a parameter changes (the reference re-stacks every call,
model.py:271,305-308).

Scope: inference (no autograd through the HIP block), one GPU.  The
``return_stats`` diagnostics (model.py:327-349) are computed with torch from
the kernels' routing outputs.  With offload_experts (Orbit Dobu) the expert
FFN weights stay in host memory behind an HBM working set (dobu.py).  Lumen
is outside this module and rejected at construction.
"""
from __future__ import annotations

import ctypes

import torch
import torch.nn.functional as F
from torch import nn

from . import _native as nat
from .config import ModelConfig
from .quant import (Int4Tensor, interleave_gate_up, interleave_gate_up_rows,
                    quantize_fp8_per_channel, quantize_int4)


class SwiGLUGate(nn.Module):
    """Marker module between the fused [gate; up] projection and W_down."""

    def forward(self, x):  # pragma: no cover - the HIP kernels apply it
        g, u = x.chunk(2, dim=-1)
        return F.silu(g) * u


# Count of parameter / submodule registrations in the process (torch's global
# registration hooks): SpiderMoELayer re-lists its parameters when it moves.
_REGISTRATIONS = [0]


def _count_registration(module, name, value):
    _REGISTRATIONS[0] += 1


torch.nn.modules.module.register_module_parameter_registration_hook(_count_registration)
torch.nn.modules.module.register_module_module_registration_hook(_count_registration)


def _share(stack: torch.Tensor, params) -> None:
    """Re-point each parameter's storage at its slice of the stacked copy the
    kernels read (same values, same shape and dtype), so the weights are
    held once, not twice.  In-place updates of a parameter then write the
    stack too and bump the parameter's version, which repacks."""
    for i, p in enumerate(params):
        if p.shape == stack[i].shape and p.dtype == stack.dtype and p.device == stack.device:
            p.data = stack[i]


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """The kernels read rows as 16-byte vectors: copy views whose storage
    offset breaks that alignment."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _Packed:
    """Device buffers in the kernels' layout + the smoe_block descriptor."""

    def __init__(self):
        self.keep = []
        self.desc = nat.SmoeBlock()
        self.ws_need = {}  # tokens -> workspace bytes


class SpiderMoELayer(nn.Module):
    """Shared recurrent layer: router + per-loop sparse graph + expert FFNs."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        if getattr(cfg, "use_lumen", False):
            raise NotImplementedError("use_lumen is not part of spider_moe_amd")
        h, e = cfg.hidden_size, cfg.num_experts
        u = cfg.expert_ffn_size
        self.num_experts, self.top_k = e, cfg.top_k
        self.top_dobu = int(getattr(cfg, "offload_max_gpu_experts", 4))
        self.edges_per_expert = cfg.edges_per_expert
        self.num_loops = cfg.num_loops
        self.loop_embed_size = cfg.loop_embed_size
        self.hidden_size = h
        self.expert_ffn_size = u
        self.expert_activation = getattr(cfg, "expert_activation", "gelu")
        self.router = nn.Linear(h, e, bias=False)
        self.loop_bias = nn.Parameter(torch.zeros(cfg.num_loops, e))
        self.loop_embedding = nn.Embedding(cfg.num_loops, cfg.loop_embed_size)
        self.edge_generator = nn.Linear(h + cfg.loop_embed_size, e * e)
        self.edge_value = nn.ModuleList([nn.Linear(h, h, bias=False) for _ in range(e)])
        if self.expert_activation == "swiglu":
            # experts.{e}.0.weight = [gate; up] stacked [2U, H]; no biases
            self.experts = nn.ModuleList([
                nn.Sequential(nn.Linear(h, 2 * u, bias=False), SwiGLUGate(),
                              nn.Linear(u, h, bias=False)) for _ in range(e)])
        else:
            self.experts = nn.ModuleList([
                nn.Sequential(nn.Linear(h, u), nn.GELU(), nn.Linear(u, h)) for _ in range(e)])
        self.norm = nn.LayerNorm(h)
        self.exit_head = nn.Linear(h, 1)
        self.residual_scale = cfg.residual_scale
        self.reinject_weight = cfg.re_inject_weight
        self.early_exit_threshold = float(getattr(cfg, "early_exit_threshold", 0.85))
        self.expert_parallel = bool(getattr(cfg, "expert_parallel", True))
        self.offload_experts = False
        self._expert_store = None
        self.lumen = None
        # quantized expert state (model.py:211-215 names for int4)
        self._int4_w_up: Int4Tensor | None = None
        self._int4_w_down: Int4Tensor | None = None
        self._int4_b_up = None
        self._int4_b_down = None
        self._fp8 = None  # (codes_up, scale_up, codes_down, scale_down)
        # bf16 / fp8 weights also get a copy in the weight tile layout
        # (lane-ordered MFMA fragments, 1 KB per 16 rows x 32 k), which the
        # decode weight stream and the prefill GEMM read with contiguous 1 KB
        # loads; int4 experts a copy of their bytes in the int4 tile layout,
        # which the prefill GEMM widens in registers.  False saves that
        # memory (same results for bf16 / fp8; int4 prefill then runs the
        # general int4 kernel)
        self.weight_tiles = True
        self._packed: _Packed | None = None
        self._packed_key = None
        self._plist = None
        self._plist_gen = -1
        self._ws: torch.Tensor | None = None
        self._last_n = 0
        self._last_ws: torch.Tensor | None = None
        self._expert_key = None
        if getattr(cfg, "offload_experts", False):
            self.enable_offload(self.top_dobu)

    # ------------------------------------------------------ Dobu offload ----
    def enable_offload(self, top_dobu: int = 4, *, pin_memory: bool = True,
                       storage_device: str = "cpu"):
        """Expert weights to a pinned host catalogue with an HBM working set
        of top_dobu experts (model.py:189-201, orbit/dobu.py:82-101); the
        expert modules leave the GPU.  Forward then runs the block's stages
        with the FFN fed from the store.  Returns the store."""
        from .dobu import ExpertChunkStore, offload_module_list_to_cpu
        if self.expert_activation != "gelu":
            raise ValueError("Dobu offload holds Linear + GELU + Linear experts")
        self.top_dobu = int(top_dobu)
        self._expert_store = ExpertChunkStore(self.experts, storage_device=storage_device,
                                              max_gpu_experts=self.top_dobu,
                                              pin_memory=pin_memory)
        self._expert_key = self._experts_key()
        offload_module_list_to_cpu(self.experts)
        self._expert_key = self._experts_key()
        self.offload_experts = True
        self._packed = None
        return self._expert_store

    def _apply(self, fn, *args, **kwargs):
        """.to() / .cuda() / .bfloat16(): offloaded experts are converted,
        copied into the catalogue and moved back to the host."""
        super()._apply(fn, *args, **kwargs)
        if self.offload_experts and self._expert_store is not None:
            self._sync_offloaded_experts()
        return self

    def _experts_key(self):
        return tuple((p.data_ptr(), p._version, p.device.type) for p in self.experts.parameters())

    def _sync_offloaded_experts(self):
        """A weight of the (offloaded) expert modules changed, or the modules
        were moved back to the GPU: refresh the catalogue, offload again."""
        from .dobu import offload_module_list_to_cpu
        key = self._experts_key()
        if key == self._expert_key:
            return
        self._expert_store.load_catalogue(self.experts)
        offload_module_list_to_cpu(self.experts)
        self._expert_key = self._experts_key()

    # ------------------------------------------------------ quantization ----
    @torch.no_grad()
    def quantize_experts(self, group_size: int = 64, scale_dtype: torch.dtype = torch.float32) -> None:
        """Group-wise INT4 expert weights (model.py:218-231); biases stay fp."""
        w_up = torch.stack([ex[0].weight.detach() for ex in self.experts], dim=0)
        w_down = torch.stack([ex[2].weight.detach() for ex in self.experts], dim=0)
        self._int4_w_up = quantize_int4(w_up, group_size=group_size, scale_dtype=scale_dtype)
        self._int4_w_down = quantize_int4(w_down, group_size=group_size, scale_dtype=scale_dtype)
        if self.expert_activation == "gelu":
            self._int4_b_up = torch.stack([ex[0].bias.detach() for ex in self.experts], dim=0)
            self._int4_b_down = torch.stack([ex[2].bias.detach() for ex in self.experts], dim=0)
        self._fp8 = None
        self._packed_key = None

    @torch.no_grad()
    def quantize_experts_fp8(self) -> None:
        """fp8-e4m3 expert weights with per-output-channel fp32 scales."""
        w_up = torch.stack([ex[0].weight.detach() for ex in self.experts], dim=0)
        w_down = torch.stack([ex[2].weight.detach() for ex in self.experts], dim=0)
        self._fp8 = (*quantize_fp8_per_channel(w_up), *quantize_fp8_per_channel(w_down))
        self._int4_w_up = self._int4_w_down = self._int4_b_up = self._int4_b_down = None
        self._packed_key = None

    def dequantize_experts(self) -> None:
        """Back to the nn.Linear weights (model.py:233-238)."""
        self._int4_w_up = self._int4_w_down = self._int4_b_up = self._int4_b_down = None
        self._fp8 = None
        self._packed_key = None

    @property
    def expert_format(self) -> str:
        if self._int4_w_up is not None:
            return "int4"
        if self._fp8 is not None:
            return "fp8"
        return "bf16" if self.router.weight.dtype == torch.bfloat16 else "f32"

    # ----------------------------------------------------------- packing ----
    def _live_params(self):
        """The layer's parameter objects.  Walking the module tree costs
        more than the pack key (~0.7 ms at 64 experts), so the list is
        cached and walked again only after a parameter or module was
        registered anywhere in the process: assigning a new nn.Parameter,
        load_state_dict(assign=True) and swapping a submodule all register
        one (_REGISTRATIONS)."""
        if self._plist is None or self._plist_gen != _REGISTRATIONS[0]:
            self._plist_gen = _REGISTRATIONS[0]
            self._plist = list(self.parameters())
        return self._plist

    def _state_key(self):
        # a parameter that is replaced, modified in place, moved (.to) or
        # re-typed changes its identity, version, address or dtype
        plist = self._live_params()
        return (self.expert_format, id(self._int4_w_up), id(self._fp8), self.weight_tiles,
                len(plist), tuple([(id(p), p.data_ptr(), p._version, p.dtype) for p in plist]))

    def _check_supported(self):
        """The shapes the HIP block takes (the reference takes any,
        model.py:165-185, config.py:41-52): a clear error before any launch."""
        e, k, m, h = self.num_experts, self.top_k, self.edges_per_expert, self.hidden_size
        bad = []
        if not 1 <= e <= 256:
            bad.append(f"num_experts {e} (1..256)")
        if not 1 <= k <= min(e, 16):
            bad.append(f"top_k {k} (1..min(num_experts, 16))")
        if not 1 <= m <= min(e, 16):
            bad.append(f"edges_per_expert {m} (1..min(num_experts, 16))")
        if min(e, k * m) > 64:
            bad.append(f"min(num_experts, top_k * edges_per_expert) = {min(e, k * m)} (<= 64)")
        if h % 8 or h > 4096:
            bad.append(f"hidden_size {h} (a multiple of 8, <= 4096)")
        if bad:
            raise ValueError("spider_moe_amd's HIP block does not take " + "; ".join(bad))

    @torch.no_grad()
    def _pack(self) -> _Packed:
        key = self._state_key()
        if self._packed is not None and self._packed_key == key:
            return self._packed
        self._check_supported()
        expert_ids = {id(p) for p in self.experts.parameters()} if self.offload_experts else set()
        dev = nat.require_gpu(*[p for p in self.parameters() if id(p) not in expert_ids])
        act = self.router.weight.dtype
        adt = nat.dtype_code(act)
        e, h, u = self.num_experts, self.hidden_size, self.expert_ffn_size
        r, lemb = self.num_loops, self.loop_embed_size
        k = _Packed()

        def keep(t):
            t = t.detach().contiguous()
            k.keep.append(t)
            return t

        def f32(t):
            return keep(t.detach().to(device=dev, dtype=torch.float32))

        swiglu = self.expert_activation == "swiglu"
        router_w = keep(self.router.weight)
        loop_bias = f32(self.loop_bias)
        edge_w = keep(self.edge_generator.weight)
        edge_b = f32(self.edge_generator.bias)
        emb = f32(self.loop_embedding.weight)
        edge_lb = keep(torch.empty(r, e * e, device=dev, dtype=torch.float32))
        edge_value = keep(torch.stack([m.weight.detach() for m in self.edge_value]))
        _share(edge_value, [m.weight for m in self.edge_value])
        lib = nat.lib()
        nat.check(lib.smoe_edge_loop_bias(edge_w.data_ptr(), adt, edge_b.data_ptr(),
                                          emb.data_ptr() if lemb > 0 else None, e, h, lemb, r,
                                          edge_lb.data_ptr(), nat.stream_of(dev)),
                  "smoe_edge_loop_bias")

        ex = nat.SmoeExperts()
        ex.E, ex.H, ex.U = e, h, u
        ex.act = nat.ACT_SWIGLU if swiglu else nat.ACT_GELU
        fmt = self.expert_format

        def gate_up(t):  # [E, 2U, X] stacked [gate; up] -> block interleave
            return interleave_gate_up(t[:, :u], t[:, u:]) if swiglu else t

        if self.offload_experts:  # the FFN weights come from the Dobu store
            ex.format = adt
            w_up = w_down = s_up = s_down = b_up = b_down = None
        elif fmt == "int4":
            qu, qd = self._int4_w_up, self._int4_w_down
            ex.format = nat.INT4
            ex.group_size = qu.group_size
            if qd.group_size != qu.group_size:
                raise RuntimeError("int4 up/down group sizes differ")
            ex.scale_dtype = nat.F16 if qu.scales.dtype == torch.float16 else nat.F32
            w_up = keep(gate_up(qu.packed.to(dev)))
            s_up = keep(gate_up(qu.scales.to(dev)))
            w_down = keep(qd.packed.to(dev))
            s_down = keep(qd.scales.to(dev))
            b_up = f32(self._int4_b_up) if self._int4_b_up is not None else None
            b_down = f32(self._int4_b_down) if self._int4_b_down is not None else None
        elif fmt == "fp8":
            cu, su, cd, sd = self._fp8
            ex.format = nat.FP8_E4M3
            ex.scale_dtype = nat.F32
            w_up = keep(gate_up(cu.to(dev).view(torch.uint8)))
            s_up = f32(interleave_gate_up_rows(su[:, :u], su[:, u:]) if swiglu else su)
            w_down = keep(cd.to(dev).view(torch.uint8))
            s_down = f32(sd)
            b_up = b_down = None
            if not swiglu:
                b_up = f32(torch.stack([m[0].bias for m in self.experts]))
                b_down = f32(torch.stack([m[2].bias for m in self.experts]))
        else:
            ex.format = adt
            w_up = keep(gate_up(torch.stack([m[0].weight.detach() for m in self.experts])))
            w_down = keep(torch.stack([m[2].weight.detach() for m in self.experts]))
            if not swiglu:  # the interleaved [gate; up] stack is not a slice per expert
                _share(w_up, [m[0].weight for m in self.experts])
            _share(w_down, [m[2].weight for m in self.experts])
            s_up = s_down = None
            b_up = b_down = None
            if not swiglu:
                b_up = f32(torch.stack([m[0].bias for m in self.experts]))
                b_down = f32(torch.stack([m[2].bias for m in self.experts]))
        ex.w_up, ex.w_down = nat.ptr(w_up), nat.ptr(w_down)
        ex.s_up, ex.s_down = nat.ptr(s_up), nat.ptr(s_down)
        ex.b_up, ex.b_down = nat.ptr(b_up), nat.ptr(b_down)

        def tiles(w, code=nat.BF16):  # copy in the weight tile layout (smoe_pack_weight_tiles)
            if w is None or not self.weight_tiles or w.shape[1] % 16 or w.shape[2] % 64:
                return None
            if w.dtype != (torch.bfloat16 if code == nat.BF16 else torch.uint8):
                return None
            out = keep(torch.empty_like(w))
            nat.check(lib.smoe_pack_weight_tiles(w.data_ptr(), code, w.shape[0], w.shape[1],
                                                 w.shape[2], out.data_ptr(), nat.stream_of(dev)),
                      "smoe_pack_weight_tiles")
            return out

        def int4_tiles(q):  # the same bytes in the int4 tile layout (smoe_pack_int4_qtiles)
            if q is None or not self.weight_tiles or q.shape[1] % 64 or (2 * q.shape[2]) % 32:
                return None
            out = keep(torch.empty_like(q))
            nat.check(lib.smoe_pack_int4_qtiles(q.data_ptr(), q.shape[0], q.shape[1], 2 * q.shape[2],
                                                out.data_ptr(), nat.stream_of(dev)),
                      "smoe_pack_int4_qtiles")
            return out

        if ex.format == nat.FP8_E4M3:
            ex.w_up_tiles = nat.ptr(tiles(w_up, nat.FP8_E4M3))
            ex.w_down_tiles = nat.ptr(tiles(w_down, nat.FP8_E4M3))
        elif ex.format == nat.INT4:
            ex.w_up_tiles = nat.ptr(int4_tiles(w_up))
            ex.w_down_tiles = nat.ptr(int4_tiles(w_down))
        elif ex.format == nat.BF16:
            ex.w_up_tiles = nat.ptr(tiles(w_up))
            ex.w_down_tiles = nat.ptr(tiles(w_down))

        d = k.desc
        d.act_dtype = adt
        d.H, d.E, d.K, d.M, d.L, d.R = h, e, self.top_k, self.edges_per_expert, lemb, r
        d.router_w, d.loop_bias = router_w.data_ptr(), loop_bias.data_ptr()
        d.edge_gen_w, d.edge_loop_bias = edge_w.data_ptr(), edge_lb.data_ptr()
        d.edge_value_w = edge_value.data_ptr()
        d.edge_value_w_tiles = nat.ptr(tiles(edge_value))
        d.experts = ex
        d.ln_w, d.ln_b = f32(self.norm.weight).data_ptr(), f32(self.norm.bias).data_ptr()
        d.alpha, d.beta, d.eps = self.residual_scale, self.reinject_weight, self.norm.eps
        # exit gate: exit_head weight [H] then bias, fp32
        k.exit_wb = f32(torch.cat([self.exit_head.weight.reshape(-1), self.exit_head.bias.reshape(-1)]))
        # the parameters that now live in the stacks moved: the key after the move
        self._packed, self._packed_key = k, self._state_key()
        return k

    def workspace_bytes(self, n: int, packed: _Packed | None = None) -> int:
        """Bytes of the native workspace a call over n tokens needs."""
        k = packed if packed is not None else self._pack()
        need = k.ws_need.get(n)
        if need is None:
            need = nat.lib().smoe_block_workspace_bytes(ctypes.byref(k.desc), n)
            if need == 0:
                nat.check(nat.lib().smoe_block_workspace_layout(ctypes.byref(k.desc), n,
                                                                ctypes.byref(nat.SmoeWsLayout())),
                          "smoe_block_workspace_layout")
            need = k.ws_need[n] = max(need, 256)
        return need

    def _workspace(self, n: int, dev, packed: _Packed) -> torch.Tensor:
        need = self.workspace_bytes(n, packed)
        if self._ws is None or self._ws.numel() < need or self._ws.device != dev:
            self._ws = torch.empty(need, dtype=torch.uint8, device=dev)
        return self._ws

    # ----------------------------------------------------------- forward ----
    def _run(self, h, x0, loop_begin: int, num_loops: int, gate=None, workspace=None):
        """workspace: a caller-owned uint8 device tensor of at least
        workspace_bytes(B*T) bytes (a captured graph keeps its own), or None
        for the layer's shared one (reallocated when a call needs more)."""
        if torch.is_grad_enabled() and self.training and any(p.requires_grad for p in self.parameters()):
            raise RuntimeError("spider_moe_amd's HIP block is forward-only: call it under "
                               "torch.no_grad() or in eval mode")
        b, t, width = h.shape
        dev = nat.require_gpu(h, x0, self.router.weight)
        act = self.router.weight.dtype
        h2 = _aligned(h.reshape(b * t, width).to(act).contiguous())
        x2 = _aligned(x0.reshape(b * t, width).to(act).contiguous())
        n = b * t
        if num_loops == 0:  # no loop to run: h unchanged (a copy, as for any call)
            return h2.clone().view(b, t, width)
        if self.offload_experts:
            return self._run_offload(h2, x2, loop_begin, num_loops, gate).view(b, t, width)
        out = torch.empty_like(h2)
        k = self._pack()
        if workspace is None:
            ws = self._workspace(n, dev, k)
        else:
            need = self.workspace_bytes(n, k)
            if (workspace.dtype != torch.uint8 or workspace.device != dev
                    or not workspace.is_contiguous() or workspace.numel() < need):
                raise ValueError("workspace must be a contiguous uint8 tensor on the input's GPU "
                                 f"of at least {need} bytes")
            ws = workspace
        if gate is None:
            nat.check(nat.lib().smoe_block_forward(ctypes.byref(k.desc), h2.data_ptr(), x2.data_ptr(),
                                                   out.data_ptr(), n, loop_begin, num_loops,
                                                   ws.data_ptr(), ws.numel(), nat.stream_of(dev)),
                      "smoe_block_forward")
        else:
            threshold, active, loops = gate
            nat.check(nat.lib().smoe_block_forward_exit(
                ctypes.byref(k.desc), h2.data_ptr(), x2.data_ptr(), out.data_ptr(), n, loop_begin,
                num_loops, k.exit_wb.data_ptr(), float(threshold), active.data_ptr(),
                loops.data_ptr(), ws.data_ptr(), ws.numel(), nat.stream_of(dev)),
                "smoe_block_forward_exit")
        self._last_n = n
        self._last_ws = ws
        return out.view(b, t, width)

    def _run_offload(self, x, x0, loop_begin: int, num_loops: int, gate=None):
        """Loops with the expert FFN from the Dobu store (model.py:294-297):
        router top-k, edge top-m and messages, the store's sparse delta, the
        residual / LayerNorm epilogue — the block's stage entry points,
        which smoe_block_forward chains inside one call.  The early-exit
        gate is applied between loops as model.py:450-473 does."""
        self._sync_offloaded_experts()
        k = self._pack()
        d = k.desc
        dev = x.device
        lib, st = nat.lib(), nat.stream_of(dev)
        n, hid = x.shape
        e, kk, m = self.num_experts, self.top_k, self.edges_per_expert
        act = d.act_dtype
        store = self._expert_store
        fdt = store.dtype
        logits = torch.empty(n, e, device=dev)
        top_w = torch.empty(n, kk, device=dev)
        top_i = torch.empty(n, kk, dtype=torch.int32, device=dev)
        eidx = torch.empty(n, kk, m, dtype=torch.int32, device=dev)
        ew = torch.empty(n, kk, m, device=dev)
        msg = torch.empty(n, hid, dtype=fdt, device=dev)

        def ws(nbytes):
            return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)

        w0 = ws(lib.smoe_router_workspace_bytes(n, e))
        w1 = ws(lib.smoe_edge_topm_workspace_bytes(n, kk, e, m))
        w2 = ws(lib.smoe_edge_message_workspace_bytes(n, hid, e, kk, m, act))
        if gate is not None:
            threshold, active, loops = gate
            exit_w = self.exit_head.weight.detach()
            exit_b = self.exit_head.bias.detach()
        for r in range(loop_begin, loop_begin + num_loops):
            nat.check(lib.smoe_router_topk(x.data_ptr(), act, n, hid, d.router_w,
                                           d.loop_bias + 4 * r * e, e, kk, logits.data_ptr(),
                                           top_w.data_ptr(), top_i.data_ptr(), w0.data_ptr(),
                                           w0.numel(), st),
                      "smoe_router_topk")
            nat.check(lib.smoe_edge_topm(x.data_ptr(), act, n, hid, d.edge_gen_w, hid + d.L,
                                         d.edge_loop_bias + 4 * r * e * e, e, kk, m,
                                         top_i.data_ptr(), eidx.data_ptr(), ew.data_ptr(),
                                         w1.data_ptr(), w1.numel(), st), "smoe_edge_topm")
            nat.check(lib.smoe_edge_message(x.data_ptr(), act, n, hid, d.edge_value_w,
                                            d.edge_value_w_tiles, e, kk, m, top_i.data_ptr(),
                                            eidx.data_ptr(), ew.data_ptr(), msg.data_ptr(),
                                            nat.dtype_code(fdt), w2.data_ptr(), w2.numel(), st),
                      "smoe_edge_message")
            delta = store.sparse_delta(msg, top_i, top_w, kk, out_dtype=torch.float32)
            out = torch.empty_like(x)
            nat.check(lib.smoe_combine_epilogue(x.data_ptr(), x0.data_ptr(), act,
                                                delta.data_ptr(), nat.F32, n, hid, d.alpha,
                                                d.beta, d.ln_w, d.ln_b, d.eps, out.data_ptr(),
                                                st), "smoe_combine_epilogue")
            if gate is not None:  # frozen rows keep h; a row leaves after the loop it passes
                on = active.bool()
                loops += on.to(torch.int32)
                out = torch.where(on.unsqueeze(-1), out, x)
                conf = torch.sigmoid(torch.nn.functional.linear(out, exit_w, exit_b).float())
                active.mul_((~(conf.squeeze(-1) > threshold)).to(torch.int32))
            x = out
        self._last_n = n
        self._offload_last = {"msg": msg, "logits": logits, "top_idx": top_i, "top_w": top_w,
                              "edge_idx": eidx.view(n * kk, m), "edge_w": ew.view(n * kk, m)}
        return x

    def forward(self, h, x0, loop_idx, return_stats=False):
        """One loop of the block (model.py:240-349)."""
        if not 0 <= int(loop_idx) < self.num_loops:
            raise IndexError(f"loop_idx {loop_idx} out of range [0, {self.num_loops})")
        updated = self._run(h, x0, int(loop_idx), 1)
        if not return_stats:
            return updated
        return updated, self._stats(h, updated, int(loop_idx))

    def forward_loops(self, h, x0, loop_begin: int = 0, num_loops: int | None = None, *,
                      workspace=None):
        """Loops [loop_begin, loop_begin+num_loops) in one native call — the
        loop driver of SpiderWebLM._run_recurrent_full (model.py:445-448).
        With num_loops == 0 the result is a copy of h."""
        if num_loops is None:
            num_loops = self.num_loops - loop_begin
        if loop_begin < 0 or num_loops < 0 or loop_begin + num_loops > self.num_loops:
            raise IndexError("loop range out of bounds")
        return self._run(h, x0, loop_begin, num_loops, workspace=workspace)

    def forward_loops_exit(self, h, x0, threshold: float | None = None, loop_begin: int = 0,
                           num_loops: int | None = None, active=None, loops=None, *,
                           workspace=None):
        """Early-exit decode over loops [loop_begin, loop_begin+num_loops)
        in one native call, the active set kept on the device
        (SpiderWebLM._run_recurrent_decode with early_exit, model.py:450-473;
        ActiveSet, active_set.py:14-64).  A token leaves the orbit after the
        loop where sigmoid(exit_head(h')) > threshold and keeps that h'.
        active / loops (int32 [B*T], updated in place; default: all in
        orbit / zeros) carry the set across calls.  threshold defaults to
        the config's early_exit_threshold.  Returns (h_out, active, loops);
        loops[t] = loops token t ran."""
        if threshold is None:
            threshold = self.early_exit_threshold
        if num_loops is None:
            num_loops = self.num_loops - loop_begin
        if loop_begin < 0 or num_loops < 0 or loop_begin + num_loops > self.num_loops:
            raise IndexError("loop range out of bounds")
        n = h.shape[0] * h.shape[1]
        if active is None:
            active = torch.ones(n, dtype=torch.int32, device=h.device)
        if loops is None:
            loops = torch.zeros(n, dtype=torch.int32, device=h.device)
        for name, t in (("active", active), ("loops", loops)):
            if t.dtype != torch.int32 or t.numel() != n or not t.is_contiguous() or t.device != h.device:
                raise ValueError(f"{name} must be a contiguous int32 tensor of {n} elements on {h.device}")
        out = self._run(h, x0, loop_begin, num_loops, gate=(threshold, active, loops),
                        workspace=workspace)
        return out, active, loops

    # ------------------------------------------------------ diagnostics ----
    def last_routing(self) -> dict:
        """Routing of the last loop computed (copies out of the workspace).
        With Dobu offload: the staged path's message, logits, top-k and
        edges (edge rows slot for slot with top_idx)."""
        if self.offload_experts:
            return {name: t.clone() for name, t in self._offload_last.items()}
        k = self._pack()
        n = self._last_n
        lay = nat.SmoeWsLayout()
        nat.check(nat.lib().smoe_block_workspace_layout(ctypes.byref(k.desc), n, ctypes.byref(lay)),
                  "smoe_block_workspace_layout")
        ws = self._last_ws
        e, kk, m, s = self.num_experts, self.top_k, self.edges_per_expert, lay.S
        h = self.hidden_size
        fdt = torch.float32 if lay.ffn_dtype == nat.F32 else torch.bfloat16

        def view(off, count, dtype):
            esz = torch.tensor([], dtype=dtype).element_size()
            return ws[off:off + count * esz].view(dtype).clone()

        out = {
            # the last loop's message [N, H] and weighted expert outputs
            # y [N*K, H] (row = expert-plan row) in the FFN dtype
            "msg": view(lay.msg, n * h, fdt).view(n, h),
            "y": view(lay.y, n * kk * h, fdt).view(n * kk, h),
            "e_tokrow": view(lay.e_tokrow, n * kk, torch.int32).view(n, kk),
            "d_acnt": view(lay.d_acnt, e, torch.int32),
            "d_roww": view(lay.d_roww, n * s, torch.float32),
            "d_tokrow": view(lay.d_tokrow, n * s, torch.int32).view(n, s),
            "logits": view(lay.logits, n * e, torch.float32).view(n, e),
            "top_idx": view(lay.top_idx, n * kk, torch.int32).view(n, kk),
            "top_w": view(lay.top_w, n * kk, torch.float32).view(n, kk),
            "tok_e": view(lay.tok_e, n * kk, torch.int32).view(n, kk),
            "tok_ew": view(lay.tok_ew, n * kk, torch.float32).view(n, kk),
            "e_cnt": view(lay.e_cnt, e, torch.int32),
            "e_acnt": view(lay.e_acnt, e, torch.int32),
            "e_off": view(lay.e_off, e + 1, torch.int32),
            "e_rows": view(lay.e_rows, n * kk, torch.int32),
            "e_roww": view(lay.e_roww, n * kk, torch.float32),
            "edge_idx": view(lay.edge_idx, n * kk * m, torch.int32).view(n * kk, m),
            "edge_w": view(lay.edge_w, n * kk * m, torch.float32).view(n * kk, m),
            "tok_d": view(lay.tok_d, n * s, torch.int32).view(n, s),
            "tok_dc": view(lay.tok_dc, n * s, torch.float32).view(n, s),
            "d_cnt": view(lay.d_cnt, e, torch.int32),
            "d_off": view(lay.d_off, e + 1, torch.int32),
            "d_rows": view(lay.d_rows, n * s, torch.int32),
        }
        return out

    @torch.no_grad()
    def _stats(self, h, updated, loop_idx):
        """model.py:327-345 from the kernels' routing; the all-source edge
        load needs every source row's top-m, recomputed here with torch."""
        r = self.last_routing()
        b, t, _ = h.shape
        e, m = self.num_experts, self.edges_per_expert
        probs = r["logits"].softmax(-1).view(b, t, e)
        load = torch.bincount(r["top_idx"].reshape(-1).long(), minlength=e).float()
        load = load / load.sum().clamp_min(1.0)
        emb = self.loop_embedding.weight[loop_idx].view(1, 1, -1).expand(b, t, -1)
        g = self.edge_generator(torch.cat([h.to(emb.dtype), emb], dim=-1)).view(b, t, e, e)
        ev, ei = g.topk(m, dim=-1)
        ew = ev.float().softmax(-1)
        edge_load = torch.bincount(ei.reshape(-1), minlength=e).float()
        edge_load = edge_load / edge_load.sum().clamp_min(1.0)
        imp = ew.new_zeros(e).scatter_add(0, ei.reshape(-1), ew.reshape(-1))
        imp = imp / imp.sum().clamp_min(1e-9)
        return {
            "router_probs": probs,
            "expert_load": load,
            "edge_load": edge_load,
            "aux_loss": e * torch.sum(load * probs.mean(dim=(0, 1))),
            "edge_loss": e * torch.sum(edge_load * imp),
            "confidence": torch.sigmoid(self.exit_head(updated).float()).squeeze(-1),
        }


# ---------------------------------------------------------------- shell ----
def _rope_tables(head_dim, max_seq, theta):
    half = head_dim // 2
    inv = 1.0 / (theta ** (torch.arange(0, half, dtype=torch.float32) / half))
    f = torch.outer(torch.arange(max_seq, dtype=torch.float32), inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos(), emb.sin()


def _apply_rope(x, cos, sin):
    t, d = x.shape[2], x.shape[3]
    c = cos[:t].to(x.dtype).view(1, 1, t, d)
    s = sin[:t].to(x.dtype).view(1, 1, t, d)
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return x * c + torch.cat([-x2, x1], dim=-1) * s


class CausalSelfAttention(nn.Module):
    """Attention of the shell layers (model.py:37-74; not a HIP kernel here)."""

    def __init__(self, hidden, heads):
        super().__init__()
        self.heads, self.hidden = heads, hidden
        self.qkv = nn.Linear(hidden, 3 * hidden, bias=False)
        self.proj = nn.Linear(hidden, hidden, bias=False)

    def forward(self, x, cos=None, sin=None):
        b, t, _ = x.shape
        q, k, v = self.qkv(x).chunk(3, dim=-1)
        q, k, v = (y.view(b, t, self.heads, -1).transpose(1, 2) for y in (q, k, v))
        if cos is not None:
            q, k = _apply_rope(q, cos, sin), _apply_rope(k, cos, sin)
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.proj(y.transpose(1, 2).contiguous().view(b, t, self.hidden))


class TransformerLayer(nn.Module):
    """model.py:134-151."""

    def __init__(self, cfg):
        super().__init__()
        h = cfg.hidden_size
        self.ln1 = nn.LayerNorm(h)
        self.attn = CausalSelfAttention(h, cfg.num_heads)
        self.ln2 = nn.LayerNorm(h)
        self.ffn = nn.Sequential(nn.Linear(h, 4 * h), nn.GELU(), nn.Linear(4 * h, h),
                                 nn.Dropout(cfg.dropout))

    def forward(self, x, cos=None, sin=None):
        x = x + self.attn(self.ln1(x), cos, sin)
        return x + self.ffn(self.ln2(x))


class SpiderWebLM(nn.Module):
    """The LM around the block (model.py:352-717, forward path only): token
    embedding, prelude / coda attention layers, the recurrent block run
    num_loops times, final LayerNorm, tied LM head."""

    def __init__(self, cfg: ModelConfig):
        super().__init__()
        cfg.validate()
        self.cfg = cfg
        self.token_embedding = nn.Embedding(cfg.vocab_size, cfg.hidden_size)
        self.position_embedding = nn.Embedding(cfg.max_seq_len, cfg.hidden_size)
        nn.init.normal_(self.position_embedding.weight, mean=0.0, std=cfg.embedding_init_std)
        nn.init.normal_(self.token_embedding.weight, mean=0.0, std=cfg.embedding_init_std)
        self.prelude = nn.ModuleList([TransformerLayer(cfg) for _ in range(cfg.num_prelude_layers)])
        self.recurrent = SpiderMoELayer(cfg)
        self.coda = nn.ModuleList([TransformerLayer(cfg) for _ in range(cfg.num_coda_layers)])
        self.final_norm = nn.LayerNorm(cfg.hidden_size)
        self.lm_head = nn.Linear(cfg.hidden_size, cfg.vocab_size, bias=False)
        self.lm_head.weight = self.token_embedding.weight
        self.use_rope = bool(cfg.use_rope)
        if self.use_rope:
            cos, sin = _rope_tables(cfg.hidden_size // cfg.num_heads, cfg.max_seq_len, cfg.rope_theta)
            self.register_buffer("rope_cos", cos, persistent=False)
            self.register_buffer("rope_sin", sin, persistent=False)

    def _run_recurrent_full(self, h, x0):
        """model.py:445-448."""
        return self.recurrent.forward_loops(h, x0, 0, self.cfg.num_loops)

    def _run_recurrent_decode(self, h, x0, early_exit):
        """model.py:450-473: with early_exit, rows whose exit_head confidence
        passes the threshold stop consuming loops (device-side active set,
        no host synchronization between loops)."""
        if not early_exit:
            return self._run_recurrent_full(h, x0)
        return self.recurrent.forward_loops_exit(h, x0, self.cfg.early_exit_threshold)[0]

    def quantize_moe_experts(self, group_size: int = 64) -> None:
        self.recurrent.quantize_experts(group_size=group_size)

    def _embed(self, ids):
        if ids.ndim != 2:
            raise ValueError("input_ids must have shape [batch, sequence]")
        if ids.shape[1] > self.cfg.max_seq_len:
            raise ValueError("input positions exceed cfg.max_seq_len")
        tok = self.token_embedding(ids)
        if self.use_rope:
            return tok
        pos = torch.arange(ids.shape[1], device=ids.device)
        return tok + self.position_embedding(pos).unsqueeze(0)

    def forward(self, input_ids, targets=None, early_exit=False, return_stats=False):
        """model.py:673-717."""
        cos = self.rope_cos if self.use_rope else None
        sin = self.rope_sin if self.use_rope else None
        x0 = self._embed(input_ids)
        h = x0
        for layer in self.prelude:
            h = layer(h, cos, sin)
        all_stats = []
        loops_used = 0
        if not early_exit and not return_stats:
            h = self.recurrent.forward_loops(h, x0, 0, self.cfg.num_loops)
            loops_used = self.cfg.num_loops
        elif not return_stats:
            # the block is token-wise, so freezing exited tokens (model.py:694-696)
            # is the device-side active set; loops run = the last token's count
            h, _, loops = self.recurrent.forward_loops_exit(h, x0, self.cfg.early_exit_threshold)
            loops_used = int(loops.max().item()) if loops.numel() else 0
        else:
            active = torch.ones(h.shape[:2], dtype=torch.bool, device=h.device)
            for loop_idx in range(self.cfg.num_loops):
                if early_exit and not bool(active.any()):
                    break
                res = self.recurrent(h, x0, loop_idx, return_stats=return_stats)
                if return_stats:
                    new_h, st = res
                    all_stats.append(st)
                else:
                    new_h = res
                if early_exit:
                    conf = torch.sigmoid(self.recurrent.exit_head(new_h).float()).squeeze(-1)
                    h = torch.where(active.unsqueeze(-1), new_h, h)
                    active = active & ~(conf > self.cfg.early_exit_threshold)
                else:
                    h = new_h
                loops_used += 1
        for layer in self.coda:
            h = layer(h, cos, sin)
        logits = self.lm_head(self.final_norm(h))
        out = {"logits": logits, "loops_used": loops_used}
        if targets is not None:
            out["loss"] = F.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1),
                                          ignore_index=-100)
        if return_stats:
            out["stats"] = all_stats
        return out


def init_normal_(module: nn.Module, generator: torch.Generator, std: float | str = 0.02) -> None:
    """Seeded re-draw of every parameter in named_parameters order: matrices
    and embeddings N(0, std), biases 0, LayerNorm weights 1, loop_bias 0.

    std="fan_in" draws each matrix N(0, 1/fan_in) instead (fan_in = its last
    dimension; embeddings N(0, 1)), so every projection of an N(0, 1) input
    is O(1): the message, the expert delta and the residual all move the
    block's output by O(1)."""
    with torch.no_grad():
        for name, p in module.named_parameters():
            if name.endswith("loop_bias"):
                p.zero_()
            elif p.ndim == 1 and (name.startswith("norm.") or ".norm." in name or "ln1" in name
                                  or "ln2" in name or "final_norm" in name):
                p.fill_(1.0 if name.endswith("weight") else 0.0)
            elif name.endswith("bias"):
                p.zero_()
            else:
                scale = std
                if std == "fan_in":
                    scale = 1.0 if "embedding" in name else p.shape[-1] ** -0.5
                p.copy_(torch.randn(p.shape, generator=generator) * scale)


__all__ = ["SpiderMoELayer", "SpiderWebLM", "TransformerLayer", "SwiGLUGate", "init_normal_"]
