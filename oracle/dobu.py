"""Oracle: Orbit Dobu residency bookkeeping (TEST INFRASTRUCTURE ONLY).

Restates ExpertChunkStore's working-set policy (spider_moe/expert_store.py:
98-112 _materialise, as sparse_delta :121-166 calls it): per step, the
experts that have a token of positive merged weight, in ascending order
(torch.unique sorts); each one is a hit (moved to the LRU end) or a miss
(a load; inserted at the end, then the least recently used are evicted
while more than max_gpu_experts are held; with max_gpu_experts 0 nothing
is held).  The FFN values are those of sparse_expert_delta
(oracle.block.expert_delta): the store only changes where the weights live.

Pins (tests/test_oracle_dobu.py): hand-worked sequences (a hit, an
eviction order, the 0 budget, a step touching more experts than the
budget) and a brute-force replay against Python's OrderedDict semantics
written out independently.
"""
from __future__ import annotations

from collections import OrderedDict

import numpy as np


def used_experts(top_i, top_w, num_experts: int) -> list[int]:
    """expert_store.py:149-158: unique ids (ascending) whose merged weight
    over the slots is > 0 for at least one token."""
    idx = np.asarray(top_i).reshape(-1, np.asarray(top_i).shape[-1])
    w = np.asarray(top_w, np.float32).reshape(idx.shape)
    out = []
    for e in sorted(set(int(v) for v in idx.reshape(-1))):
        if not 0 <= e < num_experts:
            continue
        tw = np.zeros(idx.shape[0], np.float32)
        for s in range(idx.shape[1]):
            tw = (tw + w[:, s] * (idx[:, s] == e)).astype(np.float32)
        if (tw > 0).any():
            out.append(e)
    return out


class LruTrace:
    """The store's counters and hot set after a sequence of steps."""

    def __init__(self, max_gpu_experts: int):
        self.max = max(0, int(max_gpu_experts))
        self.lru: OrderedDict[int, None] = OrderedDict()
        self.hits = self.misses = self.loads = 0

    def step(self, used: list[int]) -> None:
        for e in used:
            if e in self.lru:
                self.hits += 1
                self.lru.move_to_end(e)
                continue
            self.misses += 1
            self.loads += 1
            if self.max > 0:
                self.lru[e] = None
                while len(self.lru) > self.max:
                    self.lru.popitem(last=False)

    @property
    def hot(self) -> list[int]:
        return list(self.lru.keys())
