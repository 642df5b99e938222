"""Admission policy of ``cxldsagr_amd.serving.SessionLRU`` on the CPU (no
device work: sessions are stand-ins), after the reference's
``PrefixSessionPool`` (cache/prefix_pool.py:127-232) in its fixed-pools mode:
hits need a published session with the same signature and enough capacity
and move to the back; misses release the user's old session and then the
least recently used ones until the pages fit; an impossible request evicts
nothing; unpublished sessions never hit; discard releases immediately."""

import pytest

from cxldsagr_amd.serving import CacheBudgetExceeded, SessionLRU


class Arena:
    def __init__(self):
        self.live, self.released, self.next = set(), [], 0

    def allocate(self, capacity):
        self.next += 1
        self.live.add(self.next)
        return self.next

    def release(self, session):
        self.live.remove(session)
        self.released.append(session)


def _lru(pages):
    arena = Arena()
    return SessionLRU(pages, allocate=arena.allocate, release=arena.release), arena


def _admit(lru, key, signature="h", capacity=64 * 4):
    lease = lru.acquire(key, signature, capacity)
    if not lease.hit:
        lru.mark_ready(key)
    return lease


def test_hit_miss_and_lru_order():
    lru, arena = _lru(8)          # two sessions of 4 pages
    assert not _admit(lru, "a").hit
    assert not _admit(lru, "b").hit
    assert _admit(lru, "a").hit   # a becomes most recent
    lease = _admit(lru, "c")      # evicts b, the least recent
    assert not lease.hit and lease.evicted == ("b",)
    assert lru.keys() == ["a", "c"]
    lease = _admit(lru, "b")      # evicts a
    assert lease.evicted == ("a",) and lru.keys() == ["c", "b"]
    assert len(arena.live) == 2 and lru.evictions == 2
    assert lru.reserved_host_pages == 8 and lru.available_host_pages == 0


def test_signature_and_capacity_changes_are_misses():
    lru, arena = _lru(16)
    _admit(lru, "a", "h1", 64 * 4)
    lease = _admit(lru, "a", "h2", 64 * 4)           # another history
    assert not lease.hit and lease.evicted == ("a",)
    lease = _admit(lru, "a", "h2", 64 * 4 + 1)       # needs a fifth page
    assert not lease.hit and lease.entry.host_pages == 5
    assert _admit(lru, "a", "h2", 64 * 3).hit        # smaller request fits the cached session
    assert len(arena.live) == 1


def test_unpublished_session_never_hits():
    lru, _ = _lru(8)
    lru.acquire("a", "h", 64)
    lease = lru.acquire("a", "h", 64)
    assert not lease.hit and lease.evicted == ("a",)


def test_impossible_request_evicts_nothing():
    lru, arena = _lru(8)
    _admit(lru, "a")
    with pytest.raises(CacheBudgetExceeded):
        lru.acquire("b", "h", 64 * 9)
    assert lru.keys() == ["a"] and arena.released == []


def test_one_large_request_evicts_several_users():
    lru, arena = _lru(8)
    for key in "abcd":
        _admit(lru, key, capacity=64 * 2)
    lease = _admit(lru, "e", capacity=64 * 6)
    assert lease.evicted == ("a", "b", "c")
    assert lru.keys() == ["d", "e"] and arena.released == [1, 2, 3]


def test_discard_and_close_release_sessions():
    lru, arena = _lru(8)
    _admit(lru, "a")
    _admit(lru, "b")
    lru.discard("a")
    lru.discard("missing")
    assert "a" not in lru and arena.released == [1]
    lru.close()
    assert len(lru) == 0 and arena.live == set()
