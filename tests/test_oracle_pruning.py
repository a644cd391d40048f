"""Pins the oracle's niche-capped pruning (oracle/pruning.py) on the CPU: the reference's known
answers (reference tests/test_model.py:165-177), invariants of the rule, and the closed form the
GPU kernel computes (survivors = the capped members of smallest (depth, niche position)) equal to
the reference's round-robin loop for any niche order."""

from __future__ import annotations

import numpy as np

from oracle.pruning import niche_capped_pruning, pruned_compute_fraction


def test_reference_known_answers():
    dec = np.zeros((1, 8, 2, 2), dtype=np.int64)
    dec[0, 4:] = 1  # two niches of 4
    conf = np.array([[0.9, 0.8, 0.7, 0.6, 0.5, 0.4, 0.3, 0.2]])
    alive = np.ones((1, 8), bool)
    for order_fn in (None, lambda n, reps: [0, 1], lambda n, reps: [1, 0]):
        new = niche_capped_pruning(dec, conf, alive, 3, seed=0, event=0, order_fn=order_fn)
        assert new.sum() == 4
        assert new[0, :4].sum() == 2 and new[0, 4:].sum() == 2  # balanced across niches
        assert new[0, 0] and new[0, 4]  # the most confident member of each niche
    assert abs(pruned_compute_fraction(2) - 0.75) < 1e-9
    assert abs(pruned_compute_fraction(8) - 0.249) < 1e-3


def _closed_form(dec, conf, alive, n_cap, order):
    """The kernel's formulation for one board with an explicit niche order."""
    K = len(alive)
    idx = [k for k in range(K) if alive[k]]
    if len(idx) <= 1:
        return alive.copy()
    rep = {}
    for k in idx:
        rep[k] = next(j for j in idx if j <= k and np.array_equal(dec[j], dec[k]))
    depth = {k: sum(1 for j in idx if j != k and rep[j] == rep[k] and
                    (conf[j] > conf[k] or (conf[j] == conf[k] and j < k))) for k in idx}
    reps = sorted(set(rep.values()))
    pos = {r: order.index(reps.index(r)) for r in reps}
    capped = [k for k in idx if depth[k] < n_cap]
    keep_n = min(len(idx) // 2, len(capped))
    ranked = sorted(capped, key=lambda k: (depth[k], pos[rep[k]]))
    out = np.zeros(K, bool)
    out[ranked[:keep_n]] = True
    return out


def test_closed_form_equals_the_round_robin_loop():
    rng = np.random.default_rng(0)
    for trial in range(300):
        K = int(rng.integers(2, 24))
        pats = rng.integers(0, 1 + int(rng.integers(1, 6)), size=(K,))
        dec = np.stack([np.full((3,), p) for p in pats])[None]  # (1, K, 3)
        conf = (rng.integers(0, 4, size=(1, K)) / 4).astype(np.float32)  # ties
        alive = rng.random((1, K)) < 0.8
        n_cap = int(rng.integers(1, 4))
        n_niches = len({int(p) for p, a in zip(pats, alive[0]) if a})
        order = [int(v) for v in rng.permutation(max(n_niches, 1))]
        got = niche_capped_pruning(dec, conf, alive, n_cap, 0, 0, order_fn=lambda n, r: order)
        ref = _closed_form(dec[0], conf[0], alive[0], n_cap, order)
        assert np.array_equal(got[0], ref), trial


def test_invariants():
    rng = np.random.default_rng(1)
    N, K = 20, 16
    dec = rng.integers(0, 3, size=(N, K, 1))
    conf = rng.random((N, K)).astype(np.float32)
    alive = rng.random((N, K)) < 0.9
    new = niche_capped_pruning(dec, conf, alive, 2, seed=5, event=3)
    assert not (new & ~alive).any()  # only alive trials survive
    for n in range(N):
        a = alive[n].sum()
        if a <= 1:
            assert np.array_equal(new[n], alive[n])
            continue
        assert new[n].sum() <= a // 2
        for v in np.unique(dec[n, alive[n], 0]):
            members = np.nonzero(alive[n] & (dec[n, :, 0] == v))[0]
            kept = members[new[n, members]]
            assert len(kept) <= 2
            # a niche keeps its most confident members
            best = members[np.argsort(-conf[n, members], kind="stable")][:len(kept)]
            assert set(kept) == set(best)
