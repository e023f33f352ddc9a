"""HIP-graph replay of a fixed-R decode step of the block.

The decode runner of spider_infer/cuda_graph.py:28-130 (CudaGraphDecodeRunner)
captures one decode step per (batch, length bucket, loops) key after warm-up
runs and replays it with the inputs copied into static buffers.  Here the
captured step is the block's R loops, with or without the early-exit gate:
the gate keeps its active set on the device (smoe_block_forward_exit), so a
decode step with early exit has no host synchronization and captures whole.

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


class BlockDecodeGraph:
    """Captures SpiderMoELayer.forward_loops / forward_loops_exit per key and
    replays it.  run() returns (h_out, loops) where loops[t] is the number
    of loops token t ran (all num_loops without early exit); both are fresh
    tensors, not the static buffers."""

    def __init__(self, layer, enabled: bool = True, warmup: int = 2):
        self.layer = layer
        self.enabled = enabled
        self.warmup = warmup
        self._graphs = {}
        self.hits = 0
        self.misses = 0
        self.fallbacks = 0

    def clear(self) -> None:
        self._graphs.clear()

    def stats(self) -> dict:
        return {"graphs": len(self._graphs), "hits": self.hits, "misses": self.misses,
                "fallbacks": self.fallbacks}

    def _eager(self, h, x0, key: BlockGraphKey, active=None, loops=None):
        if key.early_exit:
            out, _, loops = self.layer.forward_loops_exit(h, x0, key.threshold, key.loop_begin,
                                                          key.num_loops, active, loops)
            return out, loops
        out = self.layer.forward_loops(h, x0, key.loop_begin, key.num_loops)
        n = h.shape[0] * h.shape[1]
        return out, torch.full((n,), key.num_loops, dtype=torch.int32, device=h.device)

    def run(self, h, x0, early_exit: bool = True, threshold: float | None = None,
            loop_begin: int = 0, num_loops: int | None = None):
        if num_loops is None:
            num_loops = self.layer.num_loops - loop_begin
        if threshold is None:
            threshold = float(getattr(self.layer, "early_exit_threshold", 0.85))
        key = BlockGraphKey(h.shape[0] * h.shape[1], loop_begin, num_loops, bool(early_exit),
                            float(threshold))
        if not self.enabled or h.device.type != "cuda":
            self.fallbacks += 1
            return self._eager(h, x0, key)
        entry = self._graphs.get(key)
        if entry is None:
            self.misses += 1
            static_h = h.detach().clone()
            static_x0 = x0.detach().clone()
            n = key.tokens
            active = torch.ones(n, dtype=torch.int32, device=h.device)
            loops = torch.zeros(n, dtype=torch.int32, device=h.device)
            # warm-up on a side stream (packing, workspace allocation), as
            # torch.cuda.graph requires
            side = torch.cuda.Stream(device=h.device)
            side.wait_stream(torch.cuda.current_stream(h.device))
            with torch.cuda.stream(side):
                for _ in range(self.warmup):
                    active.fill_(1)
                    loops.zero_()
                    self._eager(static_h, static_x0, key, active, loops)
            torch.cuda.current_stream(h.device).wait_stream(side)
            torch.cuda.synchronize(h.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                active.fill_(1)
                loops.zero_()
                out, loops_out = self._eager(static_h, static_x0, key, active, loops)
            entry = (g, static_h, static_x0, out, loops_out)
            self._graphs[key] = entry
        else:
            self.hits += 1
        g, static_h, static_x0, out, loops_out = entry
        static_h.copy_(h)
        static_x0.copy_(x0)
        g.replay()
        return out.clone(), loops_out.clone()
