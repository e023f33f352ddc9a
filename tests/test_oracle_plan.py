"""Pins for oracle/plan.py (dispatch permutation semantics)."""
import numpy as np

from oracle import plan as P


def test_reference_known_answer_forge_04():
    # tests/test_forge_04.py:18-27 of the reference
    idx = np.array([[0, 1], [1, 2]])
    w = np.array([[0.7, 0.3], [0.6, 0.4]], np.float32)
    asg, counts, perm, perm_w, row_e = P.dispatch_plan(idx, w, 4)
    assert {a[0] for a in asg} == {0, 1, 2}
    assert counts.tolist() == [1, 2, 1, 0]
    assert perm.tolist() == [0, 0, 1, 1]
    assert row_e.tolist() == [0, 1, 1, 2]
    assert np.allclose(perm_w, [0.7, 0.3, 0.6, 0.4])


def test_duplicates_merge_and_nonpositive_drop():
    idx = np.array([[1, 1], [2, 0], [3, 3], [0, 2]])
    w = np.array([[0.4, 0.6], [0.5, 0.0], [0.5, -0.5], [-1.0, 2.0]], np.float32)
    asg, counts, perm, perm_w, row_e = P.dispatch_plan(idx, w, 4)
    # expert 0: token 1 weight 0 -> dropped; token 3 weight -1 -> dropped
    # expert 1: token 0 merged 1.0; expert 2: tokens 1 (0.5) and 3 (2.0)
    # expert 3: token 2 merged 0 -> dropped
    assert counts.tolist() == [0, 1, 2, 0]
    assert perm.tolist() == [0, 1, 3]
    assert np.allclose(perm_w, [1.0, 0.5, 2.0])


def test_brute_force_enumeration():
    rng = np.random.default_rng(3)
    for trial in range(20):
        n, k, e = rng.integers(1, 40), rng.integers(1, 5), rng.integers(1, 9)
        idx = rng.integers(0, e, (n, k))
        w = rng.standard_normal((n, k)).astype(np.float32)
        w[rng.random((n, k)) < 0.2] = 0.0
        _, counts, perm, perm_w, row_e = P.dispatch_plan(idx, w, e)
        pairs = []
        for t in range(n):
            for ex in range(e):
                acc = np.float32(0.0)
                for s in range(k):
                    if idx[t, s] == ex:
                        acc = np.float32(acc + w[t, s])
                if acc > 0:
                    pairs.append((ex, t, acc))
        pairs.sort(key=lambda p: (p[0], p[1]))
        assert perm.tolist() == [p[1] for p in pairs]
        assert row_e.tolist() == [p[0] for p in pairs]
        assert np.array_equal(perm_w, np.array([p[2] for p in pairs], np.float32).reshape(-1))
        assert counts.sum() == len(pairs)


def test_planted_order_mistake_is_caught():
    """A (token, expert) ordering — a plausible mistake — differs from the
    reference's (expert, token) order on this input."""
    idx = np.array([[0, 1], [1, 0]])
    w = np.ones((2, 2), np.float32)
    _, _, perm, _, row_e = P.dispatch_plan(idx, w, 2)
    assert perm.tolist() == [0, 1, 0, 1] and row_e.tolist() == [0, 0, 1, 1]
    token_major = [0, 0, 1, 1]
    assert perm.tolist() != token_major
