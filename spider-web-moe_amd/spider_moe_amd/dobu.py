"""Orbit Dobu expert residency (spider_moe/expert_store.py:1-202,
spider_infer/orbit/dobu.py:1-127) on MI355X.

The expert FFN weights live in one pinned host catalogue (up [E,U,H],
down [E,H,U] in the experts' dtype, biases fp32).  HBM holds a slab of
2 S expert slots (S = max(top_dobu, 1): the LRU's S plus S staging slots)
in the same layout as the resident block's stacked weights, so the FFN runs
on the same grouped-GEMM kernels (smoe_expert_delta) with the slab as a
2S-expert weight set: routed expert ids are mapped to slots on the device
(smoe_remap_ids), ids of experts not in the slab to -1.

One step (ExpertChunkStore.sparse_delta):
  1. the experts with at least one token of positive merged weight, from
     the dispatch plan's counts (one small device->host copy, where the
     reference calls .unique().tolist());
  2. in ascending expert order, chunks of S experts; each expert is made
     resident exactly as the reference's _materialise does (hit: move to
     the LRU end; miss: load, insert at the end, evict the least recently
     used beyond top_dobu; with top_dobu 0 every use streams and nothing
     stays).  A miss takes the free slot freed longest ago, an eviction
     frees its slot; with S staging slots a chunk's loads never target a
     slot of the chunk before it;
  3. per chunk, the loads (asynchronous pinned-host -> HBM copies on a copy
     stream, each after the last read of its slot) overlap the previous
     chunk's FFN; the compute stream waits for them, runs the chunk's FFN
     delta over the slab (fp32) and adds it up.
top_k (router width) and top_dobu (residency) stay independent, as there.

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
        """Experts of one chunk (and LRU slots): max(top_dobu, 1)."""
        return max(self.max_gpu_experts, 1)

    @property
    def physical_slots(self) -> int:
        """Slab slots: the LRU's plus as many staging slots, so a chunk's
        loads never wait for the chunk before it (double buffering)."""
        return 2 * self.slots

    def _chunk_bytes(self) -> int:
        esz = torch.tensor([], dtype=self.dtype).element_size()
        return 2 * self.ffn * self.hidden * esz + 4 * (self.ffn + self.hidden)

    # --------------------------------------------------------------- slab ----
    def _ensure_slab(self, dev: torch.device):
        s = self._slab
        if s is not None and s["dev"] == dev:
            return s
        n, u, h = self.physical_slots, self.ffn, self.hidden
        s = {"dev": dev,
             "up": torch.empty(n, u, h, dtype=self.dtype, device=dev),
             "down": torch.empty(n, h, u, dtype=self.dtype, device=dev),
             "b_up": torch.empty(n, u, dtype=torch.float32, device=dev),
             "b_down": torch.empty(n, h, dtype=torch.float32, device=dev),
             # copies run on a stream of their own (default priority), so
             # one chunk's loads overlap the previous chunk's GEMMs
             "copy": torch.cuda.Stream(dev),
             "read_done": [None] * n}  # per slot: event after its last read
        ex = nat.SmoeExperts()
        ex.format = nat.dtype_code(self.dtype)
        ex.act = nat.ACT_GELU
        ex.E, ex.H, ex.U = n, h, u
        ex.w_up, ex.w_down = s["up"].data_ptr(), s["down"].data_ptr()
        ex.b_up, ex.b_down = s["b_up"].data_ptr(), s["b_down"].data_ptr()
        s["desc"] = ex
        self._gpu_lru.clear()  # a new slab holds nothing yet
        self._free = list(range(n))  # slots without a hot expert, oldest freed first
        self._slab = s
        return s

    def _materialise(self, expert_id: int):
        """expert_store.py:98-112 on slab slots: (slot, load needed).  A
        miss takes the free slot freed longest ago; the evicted expert's
        slot joins the free list (it may still be read by the chunk in
        flight, which the slot's event orders)."""
        if expert_id in self._gpu_lru:
            self.hits += 1
            self._gpu_lru.move_to_end(expert_id)
            return self._gpu_lru[expert_id], False
        self.misses += 1
        self.loads += 1
        slot = self._free.pop(0)
        if self.max_gpu_experts == 0:  # always stream: nothing stays hot
            self._free.append(slot)
            return slot, True
        self._gpu_lru[expert_id] = slot
        if len(self._gpu_lru) > self.max_gpu_experts:
            _, old = self._gpu_lru.popitem(last=False)
            self._free.append(old)
        return slot, True

    def release_gpu(self) -> None:
        """expert_store.py:114-118: drop the HBM working set."""
        self._gpu_lru.clear()
        if self._slab is not None:
            torch.cuda.synchronize(self._slab["dev"])
        self._slab = None
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    # ------------------------------------------------------------ compute ----
    def _buffers(self, n: int, k: int, width: int, dev):
        """Per-shape device buffers (plan, ids, partial delta, workspace)."""
        key = (n, k, width, dev)
        b = getattr(self, "_bufs", None)
        if b is not None and b["key"] == key:
            return b
        lib = nat.lib()
        e = self.num_experts
        need = lib.smoe_dispatch_workspace_bytes(n, k, e)
        dneed = lib.smoe_expert_delta_workspace_bytes(ctypes.byref(self._slab["desc"]), n, k)
        if dneed == 0:
            raise RuntimeError("smoe_expert_delta: unsupported expert shapes "
                               f"({lib.smoe_last_error().decode()})")
        i32, f32 = torch.int32, torch.float32
        nk = max(n * k, 1)
        b = {"key": key,
             "counts": torch.empty(e, dtype=i32, device=dev),
             "offsets": torch.empty(e + 1, dtype=i32, device=dev),
             "rows": torch.empty(nk, dtype=i32, device=dev),
             "roww": torch.empty(nk, dtype=f32, device=dev),
             "tokrow": torch.empty(nk, dtype=i32, device=dev),
             "plan_ws": torch.empty(max(need, 1), dtype=torch.uint8, device=dev),
             "plan_need": need,
             "slot_ids": torch.empty(nk, dtype=i32, device=dev),
             "part": torch.empty(n, width, dtype=f32, device=dev),
             "ws": torch.empty(dneed, dtype=torch.uint8, device=dev), "need": dneed}
        self._bufs = b
        return b

    def _used_experts(self, idx, w, b, dev) -> list[int]:
        """Experts with a token of positive merged weight (dispatch plan counts)."""
        n, k = idx.shape
        nat.check(nat.lib().smoe_dispatch_plan(
            idx.data_ptr(), w.data_ptr(), n, k, self.num_experts, b["counts"].data_ptr(),
            b["offsets"].data_ptr(), b["rows"].data_ptr(), b["roww"].data_ptr(),
            b["tokrow"].data_ptr(), b["plan_ws"].data_ptr(), b["plan_need"], nat.stream_of(dev)),
            "smoe_dispatch_plan")
        return torch.nonzero(b["counts"].cpu() > 0).flatten().tolist()

    @torch.no_grad()
    def sparse_delta(self, messages: torch.Tensor, top_indices: torch.Tensor,
                     top_weights: torch.Tensor, top_k: int, *, out_dtype=None) -> torch.Tensor:
        """expert_store.py:121-166: delta [B,T,H] (or [N,H]) of the routed
        experts' FFNs (Linear + bias, erf GELU, Linear + bias) times their
        merged routing weights, the weights coming from the catalogue
        through the HBM working set.  out_dtype: default messages' dtype.

        The host decides every chunk's slots first (the LRU bookkeeping),
        uploads the chunks' expert -> slot maps at once, then enqueues: per
        chunk, its loads on the copy stream (each after the last read of
        its slot), and on the compute stream a wait for them, the id remap,
        the grouped FFN over the slab and the add into the delta."""
        dev = nat.require_gpu(messages, top_indices, top_weights)
        self.compute_device = dev
        width = messages.shape[-1]
        if width != self.hidden:
            raise ValueError(f"messages width {width} != expert hidden size {self.hidden}")
        n = messages.numel() // width
        total = torch.empty(n, width, dtype=torch.float32, device=dev)
        if n == 0:
            return total.to(out_dtype or messages.dtype).view(messages.shape)
        idx = top_indices.reshape(n, top_k).to(torch.int32).contiguous()
        w = top_weights.reshape(n, top_k).to(torch.float32).contiguous()
        msg = messages.reshape(n, width).to(self.dtype).contiguous()
        slab = self._ensure_slab(dev)
        b = self._buffers(n, top_k, width, dev)
        used = self._used_experts(idx, w, b, dev)
        chunks = []
        for start in range(0, len(used), self.slots):
            chunks.append([(e, *self._materialise(e)) for e in used[start:start + self.slots]])
        if not chunks:
            return total.zero_().to(out_dtype or messages.dtype).view(messages.shape)
        smap = torch.full((len(chunks), self.num_experts), -1, dtype=torch.int32)
        for c, chunk in enumerate(chunks):
            for e, slot, _ in chunk:
                smap[c, e] = slot
        smap = smap.to(dev)
        lib = nat.lib()
        comp = torch.cuda.current_stream(dev)
        copy = slab["copy"]
        st = comp.cuda_stream
        ex = slab["desc"]
        for c, chunk in enumerate(chunks):
            loads = [(e, slot) for e, slot, load in chunk if load]
            if loads:
                with torch.cuda.stream(copy):
                    for e, slot in loads:
                        ev = slab["read_done"][slot]
                        if ev is not None:
                            copy.wait_event(ev)
                        for name in ("up", "down", "b_up", "b_down"):
                            slab[name][slot].copy_(self._cat[name][e], non_blocking=True)
                comp.wait_stream(copy)
            nat.check(lib.smoe_remap_ids(idx.data_ptr(), idx.numel(), smap[c].data_ptr(),
                                         self.num_experts, b["slot_ids"].data_ptr(), st),
                      "smoe_remap_ids")
            out = total if c == 0 else b["part"]
            nat.check(lib.smoe_expert_delta(ctypes.byref(ex), msg.data_ptr(),
                                            b["slot_ids"].data_ptr(), w.data_ptr(), n, top_k,
                                            out.data_ptr(), nat.F32, b["ws"].data_ptr(), b["need"],
                                            st), "smoe_expert_delta")
            if c > 0:
                total.add_(out)
            done = torch.cuda.Event()
            done.record(comp)
            for _, slot, _ in chunk:
                slab["read_done"][slot] = done
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
            "slab_slots": self.physical_slots,
            "slab_bytes": per * self.physical_slots if self._slab is not None else 0,
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
