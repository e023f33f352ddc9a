"""Orbit Dobu expert residency (spider_moe/expert_store.py:1-202,
spider_infer/orbit/dobu.py:1-127) on MI355X.

The expert FFN weights live in one pinned host catalogue (up [E,U,H],
down [E,H,U] in the experts' dtype, biases fp32).  HBM holds a slab of
S = max(top_dobu, 1) expert slots in the same layout as the resident
block's stacked weights, so the FFN runs on the same grouped-GEMM kernels
(smoe_expert_delta) with the slab as an S-expert weight set: routed expert
ids are mapped to slots on the device (smoe_remap_ids), ids of experts not
in the slab to -1.

One step (ExpertChunkStore.sparse_delta):
  1. the experts with at least one token of positive merged weight, from
     the dispatch plan's counts (one small device->host copy, where the
     reference calls .unique().tolist());
  2. in ascending expert order, chunks of S experts: each expert of the
     chunk is made resident exactly as the reference's _materialise does
     (hit: move to the LRU end; miss: load, insert at the end, evict the
     least recently used beyond top_dobu; with top_dobu 0 every use streams
     through a transient slot and nothing stays), a load being one
     asynchronous pinned-host -> HBM copy per weight on the compute stream
     into the slot its evicted predecessor held;
  3. the chunk's FFN delta over the slab (fp32), summed over chunks.
Stream order keeps each copy after the previous chunk's reads of its slot
and before the current chunk's.  top_k (router width) and top_dobu
(residency) stay independent, as there.

The catalogue is a snapshot of the experts' weights; the layer refreshes
it when a weight changes (the reference keeps its construction-time copy).
"""
from __future__ import annotations

import ctypes
from collections import OrderedDict
from dataclasses import dataclass

import torch
from torch import nn

from . import _native as nat


@dataclass
class ExpertChunk:
    """One expert's FFN weights (expert_store.py:22-38): views into the
    catalogue; .to() copies them."""

    w_up: torch.Tensor
    b_up: torch.Tensor
    w_down: torch.Tensor
    b_down: torch.Tensor

    def to(self, device, non_blocking: bool = True) -> "ExpertChunk":
        return ExpertChunk(*(t.to(device, non_blocking=non_blocking)
                             for t in (self.w_up, self.b_up, self.w_down, self.b_down)))


def _expert_weights(expert: nn.Module):
    """Sequential(Linear(H, U), GELU, Linear(U, H)) -> (w_up, b_up, w_down, b_down)."""
    up, down = expert[0], expert[2]
    if up.bias is None or down.bias is None or not isinstance(expert[1], nn.GELU):
        raise ValueError("Dobu expert chunks are Linear + GELU + Linear with biases "
                         "(expert_store.py:72-77)")
    return up.weight.detach(), up.bias.detach(), down.weight.detach(), down.bias.detach()


class ExpertChunkStore:
    """CPU-resident expert catalogue + an HBM LRU working set of
    max_gpu_experts (top_dobu) experts (expert_store.py:40-202)."""

    def __init__(self, experts: nn.ModuleList, *, storage_device="cpu", compute_device=None,
                 max_gpu_experts: int = 4, pin_memory: bool = True):
        self.storage_device = torch.device(storage_device)
        if self.storage_device.type != "cpu":
            raise ValueError("the Dobu catalogue lives in host memory (storage_device='cpu')")
        self.compute_device = (torch.device(compute_device) if compute_device is not None
                               else torch.device("cuda" if torch.cuda.is_available() else "cpu"))
        self.max_gpu_experts = max(0, int(max_gpu_experts))
        self.pin_memory = bool(pin_memory) and torch.cuda.is_available()
        self._gpu_lru: OrderedDict[int, int] = OrderedDict()  # expert -> slab slot
        self.hits = self.misses = self.loads = 0
        self._slab = None
        self.load_catalogue(experts)

    # ---------------------------------------------------------- catalogue ----
    @torch.no_grad()
    def load_catalogue(self, experts: nn.ModuleList) -> None:
        """(Re)build the host catalogue from the expert modules; drops the
        HBM working set (its contents would be stale)."""
        ws = [_expert_weights(ex) for ex in experts]
        if not ws:
            raise ValueError("no experts")
        u, h = ws[0][0].shape
        dt = ws[0][0].dtype
        if dt not in (torch.float32, torch.bfloat16):
            raise ValueError(f"expert weights must be float32 or bfloat16, not {dt}")
        e = len(ws)
        if self._slab is not None:
            torch.cuda.synchronize(self._slab["dev"])  # copies may still read the old catalogue
        pin = self.pin_memory

        def host(shape, dtype):
            return torch.empty(shape, dtype=dtype, pin_memory=pin)

        self._cat = {"up": host((e, u, h), dt), "down": host((e, h, u), dt),
                     "b_up": host((e, u), torch.float32), "b_down": host((e, h), torch.float32)}
        for i, (wu, bu, wd, bd) in enumerate(ws):
            if wu.shape != (u, h) or wd.shape != (h, u) or wu.dtype != dt or wd.dtype != dt:
                raise ValueError("experts differ in shape or dtype")
            self._cat["up"][i].copy_(wu)
            self._cat["down"][i].copy_(wd)
            self._cat["b_up"][i].copy_(bu)
            self._cat["b_down"][i].copy_(bd)
        self.num_experts, self.hidden, self.ffn, self.dtype = e, h, u, dt
        self._chunks = [ExpertChunk(self._cat["up"][i], self._cat["b_up"][i], self._cat["down"][i],
                                    self._cat["b_down"][i]) for i in range(e)]
        self._gpu_lru.clear()
        self._slab = None

    def __len__(self) -> int:
        return len(self._chunks)

    @property
    def slots(self) -> int:
        return max(self.max_gpu_experts, 1)

    def _chunk_bytes(self) -> int:
        esz = torch.tensor([], dtype=self.dtype).element_size()
        return 2 * self.ffn * self.hidden * esz + 4 * (self.ffn + self.hidden)

    # --------------------------------------------------------------- slab ----
    def _ensure_slab(self, dev: torch.device):
        s = self._slab
        if s is not None and s["dev"] == dev:
            return s
        n, u, h = self.slots, self.ffn, self.hidden
        s = {"dev": dev,
             "up": torch.empty(n, u, h, dtype=self.dtype, device=dev),
             "down": torch.empty(n, h, u, dtype=self.dtype, device=dev),
             "b_up": torch.empty(n, u, dtype=torch.float32, device=dev),
             "b_down": torch.empty(n, h, dtype=torch.float32, device=dev)}
        ex = nat.SmoeExperts()
        ex.format = nat.dtype_code(self.dtype)
        ex.act = nat.ACT_GELU
        ex.E, ex.H, ex.U = n, h, u
        ex.w_up, ex.w_down = s["up"].data_ptr(), s["down"].data_ptr()
        ex.b_up, ex.b_down = s["b_up"].data_ptr(), s["b_down"].data_ptr()
        s["desc"] = ex
        self._gpu_lru.clear()  # a new slab holds nothing yet
        self._slab = s
        return s

    def _load(self, expert_id: int, slot: int) -> None:
        s = self._slab
        for name in ("up", "down", "b_up", "b_down"):
            s[name][slot].copy_(self._cat[name][expert_id], non_blocking=True)
        self.loads += 1

    def _materialise(self, expert_id: int) -> int:
        """expert_store.py:98-112 on slab slots: returns the expert's slot."""
        if expert_id in self._gpu_lru:
            self.hits += 1
            self._gpu_lru.move_to_end(expert_id)
            return self._gpu_lru[expert_id]
        self.misses += 1
        if self.max_gpu_experts == 0:  # always stream: one transient slot
            self._load(expert_id, 0)
            return 0
        if len(self._gpu_lru) < self.max_gpu_experts:
            used = set(self._gpu_lru.values())
            slot = next(i for i in range(self.slots) if i not in used)
        else:  # the least recently used leaves; its slot takes the new expert
            _, slot = self._gpu_lru.popitem(last=False)
        self._load(expert_id, slot)
        self._gpu_lru[expert_id] = slot
        return slot

    def release_gpu(self) -> None:
        """expert_store.py:114-118: drop the HBM working set."""
        self._gpu_lru.clear()
        if self._slab is not None:
            torch.cuda.synchronize(self._slab["dev"])
        self._slab = None
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    # ------------------------------------------------------------ compute ----
    def _used_experts(self, idx: torch.Tensor, w: torch.Tensor, dev) -> list[int]:
        """Experts with a token of positive merged weight (dispatch plan counts)."""
        n, k = idx.shape
        e = self.num_experts
        lib = nat.lib()
        counts = torch.empty(e, dtype=torch.int32, device=dev)
        offsets = torch.empty(e + 1, dtype=torch.int32, device=dev)
        rows = torch.empty(max(n * k, 1), dtype=torch.int32, device=dev)
        roww = torch.empty(max(n * k, 1), dtype=torch.float32, device=dev)
        tokrow = torch.empty(max(n * k, 1), dtype=torch.int32, device=dev)
        need = lib.smoe_dispatch_workspace_bytes(n, k, e)
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device=dev)
        nat.check(lib.smoe_dispatch_plan(idx.data_ptr(), w.data_ptr(), n, k, e, counts.data_ptr(),
                                         offsets.data_ptr(), rows.data_ptr(), roww.data_ptr(),
                                         tokrow.data_ptr(), ws.data_ptr(), need,
                                         nat.stream_of(dev)), "smoe_dispatch_plan")
        return torch.nonzero(counts.cpu() > 0).flatten().tolist()

    @torch.no_grad()
    def sparse_delta(self, messages: torch.Tensor, top_indices: torch.Tensor,
                     top_weights: torch.Tensor, top_k: int, *, out_dtype=None) -> torch.Tensor:
        """expert_store.py:121-166: delta [B,T,H] (or [N,H]) of the routed
        experts' FFNs (Linear + bias, erf GELU, Linear + bias) times their
        merged routing weights, the weights coming from the catalogue
        through the HBM working set.  out_dtype: default messages' dtype."""
        dev = nat.require_gpu(messages, top_indices, top_weights)
        self.compute_device = dev
        width = messages.shape[-1]
        if width != self.hidden:
            raise ValueError(f"messages width {width} != expert hidden size {self.hidden}")
        n = messages.numel() // width
        idx = top_indices.reshape(n, top_k).to(torch.int32).contiguous()
        w = top_weights.reshape(n, top_k).to(torch.float32).contiguous()
        msg = messages.reshape(n, width).to(self.dtype).contiguous()
        total = torch.zeros(n, width, dtype=torch.float32, device=dev)
        if n == 0:
            return total.to(out_dtype or messages.dtype).view(messages.shape)
        used = self._used_experts(idx, w, dev)
        slab = self._ensure_slab(dev)
        lib = nat.lib()
        stream = nat.stream_of(dev)
        ex = slab["desc"]
        need = lib.smoe_expert_delta_workspace_bytes(ctypes.byref(ex), n, top_k)
        if need == 0:
            raise RuntimeError("smoe_expert_delta: unsupported expert shapes "
                               f"({lib.smoe_last_error().decode()})")
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        slot_ids = torch.empty_like(idx)
        part = torch.empty(n, width, dtype=torch.float32, device=dev)
        for start in range(0, len(used), self.slots):
            chunk = used[start:start + self.slots]
            smap = [-1] * self.num_experts
            for e in chunk:
                smap[e] = self._materialise(e)
            smap_d = torch.tensor(smap, dtype=torch.int32).to(dev)
            nat.check(lib.smoe_remap_ids(idx.data_ptr(), idx.numel(), smap_d.data_ptr(),
                                         self.num_experts, slot_ids.data_ptr(), stream),
                      "smoe_remap_ids")
            nat.check(lib.smoe_expert_delta(ctypes.byref(ex), msg.data_ptr(), slot_ids.data_ptr(),
                                            w.data_ptr(), n, top_k, part.data_ptr(), nat.F32,
                                            ws.data_ptr(), need, stream), "smoe_expert_delta")
            total.add_(part)
        return total.to(out_dtype or messages.dtype).view(messages.shape)

    def stats(self) -> dict:
        """expert_store.py:168-196."""
        per = self._chunk_bytes()
        return {
            "num_experts": len(self._chunks),
            "gpu_hot_experts": list(self._gpu_lru.keys()),
            "max_gpu_experts": self.max_gpu_experts,
            "storage_device": str(self.storage_device),
            "compute_device": str(self.compute_device),
            "storage_bytes": per * len(self._chunks),
            "gpu_working_set_bytes": per * len(self._gpu_lru),
            "hits": self.hits,
            "misses": self.misses,
            "loads": self.loads,
            "top_dobu_lru": self.max_gpu_experts,
            "policy": "dobu_residency",
        }


def offload_module_list_to_cpu(experts: nn.ModuleList) -> None:
    """expert_store.py:199-202."""
    for ex in experts:
        ex.to("cpu")


DobuChunk = ExpertChunk
DobuStore = ExpertChunkStore


@dataclass
class DobuConfig:
    """orbit/dobu.py:44-80: the residency policy, independent of top_k."""

    enabled: bool = True
    top_dobu: int = 4
    storage_device: str = "cpu"
    pin_memory: bool = True

    @property
    def max_gpu_chunks(self) -> int:
        return self.top_dobu

    def apply_to_model_config(self, model_cfg) -> None:
        model_cfg.offload_experts = bool(self.enabled)
        model_cfg.offload_max_gpu_experts = int(self.top_dobu)

    def to_dict(self) -> dict:
        return {"name": "Orbit Dobu", "enabled": self.enabled, "top_dobu": self.top_dobu,
                "top_dobu_role": "gpu_chunk_residency_lru", "storage_device": self.storage_device,
                "pin_memory": self.pin_memory,
                "note": "top_k is separate (router); top_dobu is Dobu VRAM working set"}


def enable_dobu(model, dobu_config: DobuConfig | None = None) -> DobuStore:
    """orbit/dobu.py:82-101: attach a store to model.recurrent; top_k is
    left alone."""
    cfg = dobu_config or DobuConfig()
    cfg.apply_to_model_config(model.cfg)
    return model.recurrent.enable_offload(top_dobu=cfg.top_dobu, pin_memory=cfg.pin_memory,
                                          storage_device=cfg.storage_device)


def dobu_stats(model) -> dict | None:
    """orbit/dobu.py:104-116."""
    rec = getattr(model, "recurrent", None)
    store = getattr(rec, "_expert_store", None) if rec is not None else None
    if store is None:
        return None
    st = store.stats()
    st["name"] = "Orbit Dobu"
    st["top_k"] = getattr(rec, "top_k", None)
    st["top_dobu"] = getattr(rec, "top_dobu", None) or st.get("max_gpu_experts")
    st["top_k_role"] = "router_experts_per_token"
    st["top_dobu_role"] = "gpu_chunk_residency_lru"
    return st


__all__ = ["DobuConfig", "DobuChunk", "DobuStore", "ExpertChunk", "ExpertChunkStore",
           "enable_dobu", "dobu_stats", "offload_module_list_to_cpu"]
