"""Multi-user GR serving over one shared token pool: per-user LRU admission,
transient candidate steps and committed appends with host write-back.

The reference's serial GR service (``serving/persistent.py:56-330``,
``PersistentGRRunner``) keeps the stable history of recent users between
requests in a bounded host arena (``cache/prefix_pool.py:36-330``,
``PrefixSessionPool`` in its fixed-pools mode) and runs each request's
candidate tokens as a transient step that is never committed
(``cache/README.md:86-101``). Here, for the DSA layers of this repository:

* ``SessionLRU`` - admission by host pages: a request whose user is cached
  with the same history signature and enough capacity is a hit and moves to
  the back of the LRU; otherwise the user's old session (if any) and then the
  least recently used ones are released until the new session's pages fit.
  A request larger than the whole arena raises ``CacheBudgetExceeded``
  before anything is evicted. A session is published (``mark_ready``) only
  after its history is built; a failed request discards it.
* ``GRServingRunner`` - per request: admission, history prefill on a miss
  (index K into each layer's resident index cache, KV records fp8-packed
  straight into the session's pinned host pages), the candidate step of
  every layer (``OffloadDSALayer.forward(..., transient=True)``: candidate
  records in the pool's candidate rows, ``session.written`` unchanged), and
  optionally a committed append (``transient=False``: the records are
  written back into the session's host pages and the history grows).
  Returns the per-layer outputs and the reference's request metrics
  (hit, evicted users, admission/prefix/extend times, fetched records).

Sessions released by the LRU drop their rows from every layer's pool
(``TokenPool.release_session``), so no later owner of their host pages sees
stale residency.
"""

import time
from collections import OrderedDict
from dataclasses import dataclass, field
from typing import Any, Hashable

import torch

from cxldsagr_amd.layer import OffloadDSALayer
from cxldsagr_amd.multi_user import ChunkedForward
from cxldsagr_amd.token_pool import PAGE_SIZE, RECORD_BYTES


class CacheBudgetExceeded(ValueError):
    """The requested resources cannot fit even after all users are evicted."""


@dataclass
class SessionEntry:
    session: Any
    signature: Hashable
    capacity: int
    host_pages: int
    ready: bool = False


@dataclass(frozen=True)
class SessionLease:
    entry: SessionEntry
    hit: bool
    evicted: tuple


class SessionLRU:
    """Serial LRU of user sessions over a fixed host-page arena.

    ``allocate(capacity)`` builds a session, ``release(session)`` frees it
    (after any asynchronous use). Mirrors ``PrefixSessionPool.acquire`` /
    ``mark_ready`` / ``discard`` / ``close`` (``cache/prefix_pool.py:127-232``)
    with host pages as the only budget.
    """

    def __init__(self, host_page_capacity, *, allocate, release):
        if type(host_page_capacity) is not int or host_page_capacity <= 0:
            raise ValueError("host_page_capacity must be a positive integer")
        self.host_page_capacity = host_page_capacity
        self._allocate, self._release = allocate, release
        self._entries: "OrderedDict[Hashable, SessionEntry]" = OrderedDict()
        self.evictions = 0

    def __len__(self):
        return len(self._entries)

    def __contains__(self, key):
        return key in self._entries

    @property
    def reserved_host_pages(self):
        return sum(entry.host_pages for entry in self._entries.values())

    @property
    def available_host_pages(self):
        return self.host_page_capacity - self.reserved_host_pages

    def keys(self):
        """Users from least to most recently used."""
        return list(self._entries)

    def discard(self, key):
        entry = self._entries.pop(key, None)
        if entry is not None:
            self._release(entry.session)

    def acquire(self, key, signature, capacity):
        if type(capacity) is not int or capacity <= 0:
            raise ValueError("capacity must be a positive integer")
        pages = (capacity + PAGE_SIZE - 1) // PAGE_SIZE
        # Feasibility first: a request larger than the whole arena fails here,
        # before the LRU is touched, so it evicts no other user's session.
        if pages > self.host_page_capacity:
            raise CacheBudgetExceeded(
                f"a {capacity}-token session needs {pages} host pages but the arena "
                f"holds only {self.host_page_capacity}")
        prior = self._entries.get(key)
        if (prior is not None and prior.ready and prior.signature == signature
                and prior.capacity >= capacity):
            self._entries.move_to_end(key)
            return SessionLease(prior, True, ())
        evicted = []
        if prior is not None:
            self.discard(key)
            evicted.append(key)
        while self.reserved_host_pages + pages > self.host_page_capacity:
            victim = next(iter(self._entries))
            self.discard(victim)
            evicted.append(victim)
        self.evictions += len(evicted)
        entry = SessionEntry(self._allocate(capacity), signature, capacity, pages)
        self._entries[key] = entry
        return SessionLease(entry, False, tuple(evicted))

    def mark_ready(self, key):
        self._entries[key].ready = True

    def close(self):
        for key in tuple(self._entries):
            self.discard(key)


@dataclass
class ServingResult:
    outputs: list            # per layer: bf16 [candidates, heads, 512]
    selections: list         # per layer: TokenSelection of the candidates
    metrics: dict = field(default_factory=dict)


class GRServingRunner:
    """Serial multi-user GR runner over ``len(pools)`` DSA layers.

    ``pools``: one ``TokenPool`` per layer, all with the same host arena size
    and enough candidate rows for a request's candidates. A request is a
    mapping with ``user_id``, ``signature`` (any hashable identity of the
    stable history, e.g. a token digest), ``history_tokens`` (int),
    ``history`` (a callable returning, per layer, ``(index_k bf16 [H,128],
    kv bf16 [H,576])``; called only on a miss) and ``candidates`` (per layer
    ``(index_q, index_k, weights, q, kv)`` of the candidate tokens), plus
    optional ``commit`` (append the candidates to the history instead of a
    transient step, with ``commit_signature`` the identity of the extended
    history).

    ``chunks`` > 1 runs each layer's candidate batch through
    ``multi_user.ChunkedForward``: the recall of each chunk of rows overlaps
    the indexer of the next (same outputs; the reference runner recalls after
    the whole batch's top-k).
    """

    def __init__(self, pools, *, topk=2048, scale=576 ** -0.5, chunks=1):
        if not pools:
            raise ValueError("GRServingRunner needs at least one layer pool")
        arenas = {pool.host_capacity for pool in pools}
        if len(arenas) != 1:
            raise ValueError("every layer pool must have the same host arena size")
        self.pools = list(pools)
        self.device = pools[0].device
        self.topk, self.scale = topk, scale
        self.lru = SessionLRU(pools[0].host_capacity // PAGE_SIZE, allocate=self._allocate,
                              release=self._release)
        self.visits = {}
        self.closed = False
        if type(chunks) is not int or chunks < 1:
            raise ValueError("chunks must be a positive integer")
        self.pipelines = [ChunkedForward(pool, chunks) for pool in self.pools] if chunks > 1 else None

    # ------------------------------------------------------------- sessions
    def _allocate(self, capacity):
        layers = []
        try:
            for index, pool in enumerate(self.pools):
                session = pool.allocate_session(capacity)
                # Index keys also cover a transient candidate batch.
                layers.append(OffloadDSALayer(pool, session, capacity + pool.candidate_slots,
                                              topk=self.topk, scale=self.scale, layer_idx=index))
        except BaseException:
            for layer in layers:
                layer.pool.release_session(layer.session)
            raise
        return layers

    def _release(self, layers):
        for layer in layers:
            layer.pool.release_session(layer.session)

    # ------------------------------------------------------------- requests
    def _validate(self, request):
        uid = request["user_id"]
        if not isinstance(uid, (str, int)) or isinstance(uid, bool):
            raise TypeError("user_id must be an integer or string")
        history = request["history_tokens"]
        if type(history) is not int or history <= 0:
            raise ValueError("history_tokens must be a positive integer")
        candidates = request["candidates"]
        if len(candidates) != len(self.pools):
            raise ValueError("one candidate batch per layer")
        rows = {len(batch[0]) for batch in candidates}
        if len(rows) != 1 or not next(iter(rows)):
            raise ValueError("every layer needs the same nonempty candidate batch")
        return uid, history, next(iter(rows))

    def execute(self, request):
        if self.closed:
            raise RuntimeError("runner has been closed")
        uid, history, rows = self._validate(request)
        commit = bool(request.get("commit", False))
        torch.cuda.synchronize(self.device)
        begin = time.perf_counter()
        before = [pool.metrics() for pool in self.pools]
        capacity = history + (rows if commit else 0)
        lease = self.lru.acquire(uid, request["signature"], capacity)
        layers = lease.entry.session
        try:
            admitted = time.perf_counter()
            if not lease.hit:
                per_layer = request["history"]()
                if len(per_layer) != len(layers):
                    raise ValueError("history must hold one (index_k, kv) pair per layer")
                for layer, (index_k, kv) in zip(layers, per_layer):
                    if len(index_k) != history:
                        raise ValueError("history length differs from history_tokens")
                    layer.write_history(index_k, kv)
                torch.cuda.synchronize(self.device)
                self.lru.mark_ready(uid)
            elif any(layer.written != history for layer in layers):
                raise ValueError("cached history length differs from history_tokens")
            prefixed = time.perf_counter()
            outputs, selections = [], []
            for index, (layer, batch) in enumerate(zip(layers, request["candidates"])):
                if self.pipelines is None:
                    out, selection = layer.forward(*batch, transient=not commit)
                else:
                    out, selection = self.pipelines[index].forward(layer, *batch,
                                                                   transient=not commit)
                outputs.append(out)
                selections.append(selection)
            torch.cuda.synchronize(self.device)
            for pool in self.pools:
                pool.check_status()
            finished = time.perf_counter()
        except BaseException:
            self.lru.discard(uid)
            raise
        if commit:
            # The cached history now includes the committed candidates: a later
            # request hits only under the signature the caller gives for it.
            lease.entry.signature = request.get("commit_signature", object())
        after = [pool.metrics() for pool in self.pools]
        recalled = sum(a["recalled_records"] - b["recalled_records"] for a, b in zip(after, before))
        visit = self.visits.get(uid, 0)
        self.visits[uid] = visit + 1
        metrics = {
            "user_id": uid,
            "visit_index": visit,
            "prefix_cache_hit": lease.hit,
            "evicted_users": list(lease.evicted),
            "latency_ms": (finished - begin) * 1e3,
            "admission_ms": (admitted - begin) * 1e3,
            "prefix_ms": (prefixed - admitted) * 1e3,
            "extend_ms": (finished - prefixed) * 1e3,
            "stable_prefix_tokens": history,
            "candidate_suffix_tokens": rows,
            "committed": commit,
            "recalled_records": recalled,
            "fetch_bytes": recalled * RECORD_BYTES,
            "cached_users": len(self.lru),
            "host_pages_reserved": self.lru.reserved_host_pages,
            "host_page_capacity": self.lru.host_page_capacity,
        }
        return ServingResult(outputs, selections, metrics)

    def run(self, requests):
        for request in requests:
            yield self.execute(request)

    def close(self):
        if not self.closed:
            self.closed = True
            self.lru.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
