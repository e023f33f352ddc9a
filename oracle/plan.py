"""Oracle: the dispatch plan (TEST INFRASTRUCTURE), restated in numpy.

Follows spider_infer/forge/ep/dispatch.py:56-115 (build_dispatch_plan) and the
implicit dispatch of spider_moe/sparse_experts.py:51-56:

  for each expert e ascending:
      token_w[t] = sum over slots s (in slot order) of w[t, s] * [idx[t, s] == e]
      active     = token_w > 0
      positions  = the active token indices, ascending
      weights    = token_w[positions]
  experts with no active token are omitted.

The dispatch permutation is the concatenation of ``positions`` over experts;
counts are their lengths.  Duplicate slots of one expert merge (their weights
add in slot order), and a token whose merged weight is <= 0 (or NaN) is dropped.

Pins (tests/test_oracle_plan.py): the reference's known answer
(tests/test_forge_04.py:18-27: experts {0,1,2}, expert 1 holds 2 tokens); the
duplicate-slot case (tests/test_sparse_experts_parity.py:77-98); invariants
(counts sum to the number of positive merged pairs; each expert's positions
strictly ascending); and a brute-force per-token enumeration.  No golden
plan file is committed: the known answer and the brute force pin it.
"""
from __future__ import annotations

import numpy as np


def merged_weights(idx: np.ndarray, w: np.ndarray, num_experts: int) -> np.ndarray:
    """Dense [N, E] merged weights, accumulated in slot order in float32."""
    idx = np.asarray(idx).reshape(-1, np.asarray(idx).shape[-1])
    w = np.asarray(w, dtype=np.float32).reshape(idx.shape)
    n, k = idx.shape
    tw = np.zeros((n, num_experts), dtype=np.float32)
    for s in range(k):
        for e in range(num_experts):
            tw[:, e] = tw[:, e] + w[:, s] * (idx[:, s] == e).astype(np.float32)
    return tw


def dispatch_plan(idx: np.ndarray, w: np.ndarray, num_experts: int):
    """Return (assignments, counts[E], perm, perm_weights, expert_of_row).

    assignments: list of (expert_id, positions int64[n_e], weights f32[n_e]),
    non-empty experts only, ascending expert id.
    """
    tw = merged_weights(idx, w, num_experts)
    assignments = []
    counts = np.zeros(num_experts, dtype=np.int64)
    for e in range(num_experts):
        active = tw[:, e] > 0
        if not active.any():
            continue
        pos = np.nonzero(active)[0].astype(np.int64)
        assignments.append((e, pos, tw[pos, e].copy()))
        counts[e] = pos.size
    if assignments:
        perm = np.concatenate([a[1] for a in assignments])
        perm_w = np.concatenate([a[2] for a in assignments])
        row_e = np.concatenate([np.full(a[1].size, a[0], np.int64) for a in assignments])
    else:
        perm = np.zeros(0, np.int64)
        perm_w = np.zeros(0, np.float32)
        row_e = np.zeros(0, np.int64)
    return assignments, counts, perm, perm_w, row_e
