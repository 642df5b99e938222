"""A10/A11: exact recall into a bounded HBM token pool (TEST INFRASTRUCTURE ONLY).

Restates, for one layer of the shared pool, ``SparseTokenCache.ensure``
(``cache/sparse_token_cache.py:502-569``), its victim choice
``_available_slots`` / ``_evict`` (``:465-500``), the pool's FIFO events
``stamp`` / ``protect`` (``cache/sparse_token_pool.py:648-676``) and the CPU
gather ``records[chosen] = host[missing]`` (``sparse_token_cache.py:541-542``):

1. the union of selected ids ``>= 0``; ids at or beyond ``written`` are an
   error; history ids (below ``transient_start`` when a transient candidate
   suffix is active) beyond ``slots`` in number raise ``WorkingSetTooLarge``;
2. logical -> global host id through the session page table
   (``page_table[t // 64] * 64 + t % 64``, ``sparse_token_cache.py:203-215``);
3. misses are the union ids whose ``h2d`` is MISSING, in ascending logical
   order; hits get ``priority = clock`` and the clock advances (protect);
4. victims: slots other than the sentinel 0 and this selection's hits,
   ordered by (rank, slot) with rank -1 for empty slots and the priority
   otherwise (a stable argsort); the first ``len(misses)`` are evicted (the
   old owner's ``h2d`` becomes MISSING) and receive the misses in order;
5. gather, publish ``h2d/d2h``, stamp the chosen slots with the next clock
   value (the clock advances even when nothing was missing);
6. physical ids: ``h2d`` of each history id, ``slots + 1 + id -
   transient_start`` for candidate ids, ``-1`` for padding.

``release_ids`` restates the pool's release of a session's host rows
(``cache/sparse_token_pool.py:697-710``): resident rows free their slots
(``d2h`` MISSING, priority -1) and become MISSING in ``h2d``.

Pinned by ``tests/test_oracle_recall.py``: the reference's recall known
answer (``cache/tests/test_sparse_token_cache.py:9-36``), its map invariants
(``cache/tests/test_sparse_token_pool.py:32-44``) and its independent
free-first/minimum-priority victim-legality check
(``cache/tests/test_sparse_recall_metadata.py:117-135``) over seeded random
selection sequences; ``release_ids`` by the same map invariants after
releases, by releasing rows that are not resident (no change) and by a
recall after a release, which must fetch every released row again.
"""

import numpy as np

MISSING = 2**31 - 1
PAGE_SIZE = 64


class WorkingSetTooLarge(ValueError):
    """The caller must split query consumption without changing its selection."""


class Pool:
    """One layer: host arena, device records, maps, priorities and the FIFO clock."""

    def __init__(self, host_rows, slots, width, candidate_slots=0):
        self.slots = slots
        self.host = np.zeros((host_rows, width), np.uint8)
        self.records = np.zeros((slots + 1 + candidate_slots, width), np.uint8)
        self.h2d = np.full(host_rows, MISSING, np.int64)
        self.d2h = np.full(slots + 1, MISSING, np.int64)
        self.priority = np.full(slots + 1, -1, np.int64)
        self.priority[0] = MISSING
        self.clock = 0
        self.recalled = 0
        self.evicted = 0

    def copy(self):
        other = Pool.__new__(Pool)
        for name, value in self.__dict__.items():
            setattr(other, name, value.copy() if isinstance(value, np.ndarray) else value)
        return other

    def stamp(self, physical):
        self.priority[physical] = self.clock
        self.priority[0] = MISSING
        self.clock += 1

    def available_slots(self, protected_physical, count):
        keep = np.zeros(self.slots + 1, bool)
        keep[0] = True
        keep[protected_physical] = True
        available = np.nonzero(~keep)[0]
        if available.size < count:
            raise WorkingSetTooLarge("protected records exceed the device working set")
        rank = np.where(self.d2h[available] == MISSING, -1, self.priority[available])
        chosen = available[np.argsort(rank, kind="stable")[:count]]
        old = self.d2h[chosen]
        valid = old != MISSING
        self.h2d[old[valid]] = MISSING
        self.d2h[chosen] = MISSING
        self.priority[chosen] = -1
        self.evicted += int(valid.sum())
        return chosen


def logical_to_global(page_table, ids):
    ids = np.asarray(ids, np.int64)
    return np.asarray(page_table, np.int64)[ids // PAGE_SIZE] * PAGE_SIZE + ids % PAGE_SIZE


def ensure(pool, indices, page_table, written, transient_start=None):
    """Exact recall of ``indices [Q,K]`` (logical, -1 padding); returns int32 physical ids."""
    indices = np.asarray(indices, np.int64)
    unique = np.unique(indices)
    unique = unique[unique >= 0]
    if unique.size and unique[-1] >= written:
        raise ValueError("selection references unwritten cache records")
    history = unique if transient_start is None else unique[unique < transient_start]
    if history.size > pool.slots:
        raise WorkingSetTooLarge(f"{history.size} selected history records exceed {pool.slots} slots")
    global_ids = logical_to_global(page_table, history)
    mapped = pool.h2d[global_ids]
    missing = global_ids[mapped == MISSING]
    hits = mapped[mapped != MISSING]
    pool.stamp(hits)  # protect
    if missing.size:
        chosen = pool.available_slots(hits, missing.size)
        pool.records[chosen] = pool.host[missing]
        pool.h2d[missing] = chosen
        pool.d2h[chosen] = missing
        pool.recalled += int(missing.size)
    else:
        chosen = np.zeros(0, np.int64)
    pool.stamp(chosen)
    physical = np.full(indices.shape, -1, np.int64)
    if transient_start is None:
        valid = indices >= 0
        physical[valid] = pool.h2d[logical_to_global(page_table, indices[valid])]
    else:
        hist = (indices >= 0) & (indices < transient_start)
        physical[hist] = pool.h2d[logical_to_global(page_table, indices[hist])]
        cand = indices >= transient_start
        physical[cand] = pool.slots + 1 + indices[cand] - transient_start
    return physical.astype(np.int32)


def check_maps(pool):
    """Map invariants of the reference pool (``test_sparse_token_pool.py:32-44``)."""
    assert pool.d2h[0] == MISSING and pool.priority[0] == MISSING
    live = np.nonzero(pool.d2h != MISSING)[0]
    assert np.array_equal(pool.h2d[pool.d2h[live]], live)
    host_live = np.nonzero(pool.h2d != MISSING)[0]
    assert np.array_equal(pool.d2h[pool.h2d[host_live]], host_live)
    free = pool.d2h[1:] == MISSING
    assert (pool.priority[1:][free] == -1).all()
    assert (pool.priority[live] < pool.clock).all()
    assert np.array_equal(pool.records[live], pool.host[pool.d2h[live]])


def release_ids(pool, global_ids):
    """Free the slots of resident host rows ``global_ids`` and unmap them."""
    global_ids = np.asarray(global_ids, np.int64)
    physical = pool.h2d[global_ids]
    physical = physical[physical != MISSING]
    pool.h2d[global_ids] = MISSING
    pool.d2h[physical] = MISSING
    pool.priority[physical] = -1
