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


def test_release_ids_frees_slots_and_forces_a_fresh_recall():
    """release_ids (cache/sparse_token_pool.py:697-710): the released rows
    leave h2d and their slots become free (d2h MISSING, priority -1), the map
    invariants hold, rows that were not resident change nothing, other
    sessions' residency is kept, and a recall of the released rows fetches
    every one of them again into free slots."""
    rng = np.random.default_rng(7)
    pool = _pool_with_history(4 * 64, 128, seed=7)
    table_a, table_b = np.array([0, 1]), np.array([2, 3])
    sel_a = rng.integers(0, 128, (2, 30))
    sel_b = rng.integers(0, 128, (2, 30))
    recall.ensure(pool, sel_a, table_a, written=128)
    recall.ensure(pool, sel_b, table_b, written=128)
    b_rows = recall.logical_to_global(table_b, np.unique(sel_b))
    b_slots = pool.h2d[b_rows].copy()
    a_rows = recall.logical_to_global(table_a, np.arange(128))
    resident_a = a_rows[pool.h2d[a_rows] != recall.MISSING]
    freed = pool.h2d[resident_a].copy()
    assert resident_a.size == np.unique(sel_a).size

    recall.release_ids(pool, a_rows)
    assert (pool.h2d[a_rows] == recall.MISSING).all()
    assert (pool.d2h[freed] == recall.MISSING).all() and (pool.priority[freed] == -1).all()
    np.testing.assert_array_equal(pool.h2d[b_rows], b_slots)
    recall.check_maps(pool)

    snapshot = pool.copy()
    recall.release_ids(pool, a_rows)   # nothing resident any more: no change
    for name in ("h2d", "d2h", "priority"):
        np.testing.assert_array_equal(getattr(pool, name), getattr(snapshot, name))

    before = pool.recalled
    recall.ensure(pool, sel_a, table_a, written=128)
    assert pool.recalled - before == np.unique(sel_a).size
    assert set(pool.h2d[resident_a].tolist()) <= set(freed.tolist()) | set(
        np.nonzero(snapshot.d2h == recall.MISSING)[0].tolist())
    recall.check_maps(pool)
