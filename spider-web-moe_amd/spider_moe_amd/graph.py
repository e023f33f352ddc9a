"""HIP-graph replay of a fixed-R decode step of the block.

The decode runner of spider_infer/cuda_graph.py:28-130 (CudaGraphDecodeRunner)
captures one decode step per (batch, length bucket, loops) key after warm-up
runs and replays it with the inputs copied into static buffers.  Here the
captured step is the block's R loops, with or without the early-exit gate:
the gate keeps its active set on the device (smoe_block_forward_exit), so a
decode step with early exit has no host synchronization and captures whole.

A captured graph holds device addresses: its static inputs and outputs, the
native workspace and every packed weight buffer.  Each cache entry therefore
owns all of them: the graph gets a workspace of its own (not the layer's
shared one, which a larger eager call would reallocate), and the entry keeps
the packed parameter set it was captured against alive.  A parameter update
repacks the layer's weights into new buffers; an entry whose packed set is
no longer the layer's current one is dropped and captured again.

Inside the capture the active set is reset by fill kernels (fill_ / zero_),
not by memset nodes.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class BlockGraphKey:
    tokens: int
    loop_begin: int
    num_loops: int
    early_exit: bool
    threshold: float


@dataclass
class _Entry:
    graph: torch.cuda.CUDAGraph
    static_h: torch.Tensor
    static_x0: torch.Tensor
    out: torch.Tensor
    loops: torch.Tensor
    workspace: torch.Tensor   # the graph's own native workspace
    packed: object            # the layer's packed weights the graph reads
    packed_key: object        # the parameter state they were packed from


class BlockDecodeGraph:
    """Captures SpiderMoELayer.forward_loops / forward_loops_exit per key and
    replays it.  run() returns (h_out, loops) where loops[t] is the number
    of loops token t ran (all num_loops without early exit); both are fresh
    tensors, not the static buffers."""

    def __init__(self, layer, enabled: bool = True, warmup: int = 2):
        self.layer = layer
        self.enabled = enabled
        self.warmup = warmup
        self._graphs: dict[BlockGraphKey, _Entry] = {}
        self.hits = 0
        self.misses = 0
        self.recaptures = 0
        self.fallbacks = 0

    def clear(self) -> None:
        self._graphs.clear()

    def stats(self) -> dict:
        return {"graphs": len(self._graphs), "hits": self.hits, "misses": self.misses,
                "recaptures": self.recaptures, "fallbacks": self.fallbacks}

    def _eager(self, h, x0, key: BlockGraphKey, active=None, loops=None, workspace=None):
        if key.early_exit:
            out, _, loops = self.layer.forward_loops_exit(h, x0, key.threshold, key.loop_begin,
                                                          key.num_loops, active, loops,
                                                          workspace=workspace)
            return out, loops
        out = self.layer.forward_loops(h, x0, key.loop_begin, key.num_loops, workspace=workspace)
        n = h.shape[0] * h.shape[1]
        return out, torch.full((n,), key.num_loops, dtype=torch.int32, device=h.device)

    def _capture(self, h, x0, key: BlockGraphKey) -> _Entry:
        layer = self.layer
        static_h = h.detach().clone()
        static_x0 = x0.detach().clone()
        n = key.tokens
        packed = layer._pack()
        packed_key = layer._packed_key
        ws = torch.empty(layer.workspace_bytes(n), dtype=torch.uint8, device=h.device)
        active = torch.ones(n, dtype=torch.int32, device=h.device)
        loops = torch.zeros(n, dtype=torch.int32, device=h.device)
        # warm-up on a side stream, as torch.cuda.graph requires
        side = torch.cuda.Stream(device=h.device)
        side.wait_stream(torch.cuda.current_stream(h.device))
        with torch.cuda.stream(side):
            for _ in range(self.warmup):
                active.fill_(1)
                loops.zero_()
                self._eager(static_h, static_x0, key, active, loops, ws)
        torch.cuda.current_stream(h.device).wait_stream(side)
        torch.cuda.synchronize(h.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            active.fill_(1)
            loops.zero_()
            out, loops_out = self._eager(static_h, static_x0, key, active, loops, ws)
        if layer._packed is not packed:
            raise RuntimeError("the layer's parameters changed during graph capture")
        return _Entry(g, static_h, static_x0, out, loops_out, ws, packed, packed_key)

    def run(self, h, x0, early_exit: bool = True, threshold: float | None = None,
            loop_begin: int = 0, num_loops: int | None = None):
        if num_loops is None:
            num_loops = self.layer.num_loops - loop_begin
        if threshold is None:
            threshold = self.layer.early_exit_threshold
        key = BlockGraphKey(h.shape[0] * h.shape[1], loop_begin, num_loops, bool(early_exit),
                            float(threshold))
        if not self.enabled or h.device.type != "cuda":
            self.fallbacks += 1
            return self._eager(h, x0, key)
        entry = self._graphs.get(key)
        if entry is not None and self.layer._pack() is not entry.packed:
            # the parameters were repacked since the capture: the graph reads
            # the old weights, so capture again against the current ones
            del self._graphs[key]
            entry = None
            self.recaptures += 1
        if entry is None:
            self.misses += 1
            entry = self._capture(h, x0, key)
            self._graphs[key] = entry
        else:
            self.hits += 1
        entry.static_h.copy_(h)
        entry.static_x0.copy_(x0)
        entry.graph.replay()
        return entry.out.clone(), entry.loops.clone()
