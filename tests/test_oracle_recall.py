"""Pins of the oracle's exact recall (A10/A11), CPU only.

* the reference's recall known answer (cache/tests/test_sparse_token_cache.py:9-36):
  recalled records equal the source, padding stays -1, oversize selections
  raise WorkingSetTooLarge, unwritten ids raise;
* the pool's map invariants (cache/tests/test_sparse_token_pool.py:32-44);
* the reference's independent victim-legality check
  (cache/tests/test_sparse_recall_metadata.py:117-135): chosen slots are
  unique, never the sentinel or a protected hit, and their ranks are the
  smallest available ranks (free first, then lowest priority).
"""

import numpy as np
import pytest

from oracle import recall


def _pool_with_history(tokens, slots, width=16, candidates=0, seed=0):
    rng = np.random.default_rng(seed)
    pool = recall.Pool(tokens, slots, width, candidates)
    pool.host[:] = rng.integers(0, 256, pool.host.shape, dtype=np.uint8)
    return pool


def test_known_answer_recall_eviction_and_errors():
    pool = _pool_with_history(64, 4)
    table = np.arange(1)
    for selection in ([0, 3, 2], [3, 6, 7], [-1, 0, 6]):
        logical = np.array([selection])
        physical = recall.ensure(pool, logical, table, written=8)
        valid = logical >= 0
        assert np.array_equal(pool.records[physical[valid]], pool.host[logical[valid]])
        assert (physical[~valid] == -1).all()
        recall.check_maps(pool)
    with pytest.raises(ValueError, match="unwritten"):
        recall.ensure(pool, np.array([[8]]), table, written=8)
    with pytest.raises(recall.WorkingSetTooLarge):
        recall.ensure(pool, np.arange(5)[None], table, written=8)


def _legal(before, protected, chosen):
    chosen = [int(s) for s in chosen]
    assert len(set(chosen)) == len(chosen), "duplicate allocation slot"
    eligible = set(range(1, len(before.d2h))) - set(int(p) for p in protected)
    assert set(chosen) <= eligible, "allocation used padding/protected/out-of-range slot"
    ranks = {s: -1 if before.d2h[s] == recall.MISSING else int(before.priority[s]) for s in eligible}
    ordered = sorted(ranks.values())
    assert sorted(ranks[s] for s in chosen) == ordered[: len(chosen)], "victim order violated"


@pytest.mark.parametrize("seed", range(6))
def test_random_sequences_keep_maps_and_legal_victims(seed):
    rng = np.random.default_rng(seed)
    pages = 8
    pool = _pool_with_history(pages * 64, 128, candidates=8, seed=seed)
    table = rng.permutation(pages)
    written = pages * 64
    for step in range(12):
        q, k = rng.integers(1, 4), rng.integers(1, 40)
        sel = rng.integers(-3, written, (q, k))
        before = pool.copy()
        logical = np.unique(sel[sel >= 0])
        g = recall.logical_to_global(table, logical)
        hits = before.h2d[g][before.h2d[g] != recall.MISSING]
        missing = g[before.h2d[g] == recall.MISSING]
        physical = recall.ensure(pool, sel, table, written)
        chosen = pool.h2d[missing]
        _legal(before, hits, chosen)
        # misses are assigned in ascending logical order to slots in (rank, slot) order
        ranks = [(-1 if before.d2h[s] == recall.MISSING else before.priority[s], s) for s in chosen]
        assert ranks == sorted(ranks)
        recall.check_maps(pool)
        valid = sel >= 0
        assert np.array_equal(pool.records[physical[valid]],
                              pool.host[recall.logical_to_global(table, sel[valid])])
        assert pool.clock == 2 * (step + 1)


def test_transient_candidates_map_to_tail_rows():
    pool = _pool_with_history(128, 16, candidates=4)
    table = np.arange(2)
    sel = np.array([[0, 100, 101, -1, 103]])
    physical = recall.ensure(pool, sel, table, written=104, transient_start=100)
    assert physical[0, 1:].tolist() == [17, 18, -1, 20]
    assert np.array_equal(pool.records[physical[0, 0]], pool.host[0])
