"""Bounded HBM token pool with a pinned-host arena and exact top-k-driven recall.

The part of the reference's ``SharedSparseTokenPool`` / ``SparseTokenCache``
(``cache/sparse_token_pool.py:98-279``, ``cache/sparse_token_cache.py:33-739``)
that the DSA prefill path uses, for one layer:

* a pinned host arena of 656-byte fp8 records in 64-token pages, sessions own
  pages through a page table (``sparse_token_pool.py:170-279``);
* a device pool of ``slots`` records plus the sentinel row 0 and
  ``candidate_slots`` transient candidate rows after it;
* maps ``h2d`` (int32, MISSING = INT32_MAX), ``d2h`` and FIFO ``priority``
  (int64, -1 free, sentinel MISSING) and the host-side FIFO clock;
* ``ensure`` = exact recall of a selection (``sparse_token_cache.py:502-569``)
  run entirely on the GPU (``csrc/recall.hip``), returning physical ids for
  ``sparse_mla_fp8_paged`` over the pool (addressed through an identity page
  table).

Replaces the reference's fused ECHO prefetch: records are fetched after the
exact top-k, only for the selected tokens that are not resident.
"""

import torch

from cxldsagr_amd import _native, attention

MISSING = 2**31 - 1
PAGE_SIZE = 64
RECORD_BYTES = attention.RECORD_BYTES


class WorkingSetTooLarge(ValueError):
    """The caller must split query consumption without changing its selection."""


class Session:
    """Host pages of one sequence (``page_table[t // 64]`` is the host page of token t)."""

    def __init__(self, pool, pages):
        self.pool = pool
        self.host_pages = pages
        self.capacity = len(pages) * PAGE_SIZE
        self.page_table = torch.tensor(pages, dtype=torch.int32, device=pool.device)
        self.written = 0
        self.released = False

    def global_rows(self, start, stop):
        t = torch.arange(start, stop, dtype=torch.int64)
        pages = torch.tensor(self.host_pages, dtype=torch.int64)
        return pages[t // PAGE_SIZE] * PAGE_SIZE + t % PAGE_SIZE


class TokenPool:
    """One layer's HBM token pool over a pinned host arena of fp8 KV records."""

    def __init__(self, host_capacity, slots, *, device, candidate_slots=0, history_capacity=None):
        if type(host_capacity) is not int or host_capacity < PAGE_SIZE or host_capacity % PAGE_SIZE:
            raise ValueError("host_capacity must be a positive multiple of 64 tokens")
        if type(slots) is not int or slots < 1 or slots + candidate_slots >= MISSING:
            raise ValueError("slots must be a positive integer that fits the int32 map domain")
        if host_capacity >= MISSING:
            raise ValueError("host ids must fit the int32 mapping domain")
        self.device = torch.device(device)
        _native.require_gfx950(self.device, "token pool recall")
        self.host_capacity, self.slots, self.candidate_slots = host_capacity, slots, candidate_slots
        self.history_capacity = host_capacity if history_capacity is None else history_capacity
        self.host = torch.zeros((host_capacity, RECORD_BYTES), dtype=torch.uint8, pin_memory=True)
        rows = slots + 1 + candidate_slots
        self.record_pages = (rows + PAGE_SIZE - 1) // PAGE_SIZE
        self.records = torch.zeros((self.record_pages, PAGE_SIZE, RECORD_BYTES), dtype=torch.uint8,
                                   device=self.device)
        self.identity_pages = torch.arange(self.record_pages, dtype=torch.int32, device=self.device)
        self.h2d = torch.full((host_capacity,), MISSING, dtype=torch.int32, device=self.device)
        self.d2h = torch.full((slots + 1,), MISSING, dtype=torch.int64, device=self.device)
        self.priority = torch.full((slots + 1,), -1, dtype=torch.int64, device=self.device)
        self.priority[0] = MISSING
        self.clock = 0
        self.last_stamp = None  # protect stamp of the latest recall
        self._second_workspace = None  # for recalls whose copy runs on a gather stream
        self._parity = 0
        nbytes = _native.ctypes.c_int64(0)
        _native.call("dsa_pool_workspace_bytes", slots, self.history_capacity,
                     _native.ctypes.byref(nbytes))
        self.workspace = torch.empty(nbytes.value, dtype=torch.uint8, device=self.device)
        # union, recalled, evicted, spare (cumulative, on the device)
        self.stats = torch.zeros(4, dtype=torch.int64, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._free_pages = list(range(host_capacity // PAGE_SIZE - 1, -1, -1))

    # ------------------------------------------------------------- sessions
    def allocate_session(self, capacity):
        if type(capacity) is not int or capacity < 1:
            raise ValueError("capacity must be a positive integer")
        pages = (capacity + PAGE_SIZE - 1) // PAGE_SIZE
        if pages > len(self._free_pages):
            raise ValueError("host arena has too few free pages for this session")
        return Session(self, [self._free_pages.pop() for _ in range(pages)])

    def write_history(self, session, kv_bf16):
        """Append bf16 ``[T, 576]`` history records to the session's host pages
        and wait for them (``append_records`` followed by a synchronisation
        of the current stream: a setup path, after which the host arena may be
        read on the CPU)."""
        start = self.append_records(session, kv_bf16)
        torch.cuda.current_stream(self.device).synchronize()
        return start

    def append_records(self, session, kv_bf16):
        """Persistent append with write-back: bf16 ``[T, 576]`` records are
        quantised into the 656-byte format and stored straight into the
        session's pinned host pages by the pack kernel (zero-copy over PCIe,
        on the current stream, no staging buffer and no host
        synchronisation). The role of the reference's D2H write-back of
        appended KV (``cache/sparse_token_pool.py:468-510``, a copy-stream
        ``write_host`` that readers wait for): here the write is ordered on
        the stream before any later recall that reads those rows. CPU reads of
        ``host`` must synchronise first. Returns the first appended position.
        """
        self._check_live(session)
        start, stop = session.written, session.written + len(kv_bf16)
        if stop > session.capacity or stop > self.history_capacity:
            raise ValueError("history exceeds the session capacity")
        if (kv_bf16.dtype != torch.bfloat16 or kv_bf16.ndim != 2
                or kv_bf16.shape[1] != attention.QK_DIM or kv_bf16.device != self.device):
            raise ValueError(f"kv must be BF16 [T, {attention.QK_DIM}] on {self.device}")
        if len(kv_bf16):
            kv = kv_bf16.contiguous()
            if kv.data_ptr() % 16:
                kv = kv.clone()
            with torch.cuda.device(self.device):
                _native.call("dsa_kv_pack_fp8", _native.ptr(kv), len(kv), start,
                             _native.ptr(session.page_table), self.host_capacity // PAGE_SIZE,
                             _native.ptr(self.host), _native.ptr(self.status),
                             _native.stream_of(self.device))
        session.written = stop
        return start

    def release_session(self, session):
        """Return a session's host pages to the arena and drop its rows from
        the pool (``SharedSparseTokenPool.release_session`` /
        ``release_ids``, ``cache/sparse_token_pool.py:697-780``): every
        resident row frees its slot, so a later owner of the pages never sees
        stale residency. Synchronises the current stream (the pool must be
        quiescent, as in the reference)."""
        self._check_live(session)
        with torch.cuda.device(self.device):
            _native.call("dsa_pool_release_rows", _native.ptr(session.page_table),
                         len(session.host_pages), self.host_capacity, _native.ptr(self.h2d),
                         _native.ptr(self.d2h), _native.ptr(self.priority), self.slots,
                         _native.ptr(self.status), _native.stream_of(self.device))
            torch.cuda.current_stream(self.device).synchronize()
        self._free_pages.extend(reversed(session.host_pages))
        session.released = True
        session.written = 0

    @property
    def free_host_pages(self):
        return len(self._free_pages)

    def _check_live(self, session):
        if session.pool is not self or session.released:
            raise ValueError("session is released or belongs to another pool")

    def write_candidates(self, kv_bf16, offset=0):
        """Quantise transient candidate records into rows ``slots + 1 + offset ...``."""
        if offset < 0 or offset + len(kv_bf16) > self.candidate_slots:
            raise ValueError("candidates exceed the candidate rows")
        attention.pack_kv_fp8(kv_bf16, self.records, self.identity_pages,
                              token_offset=self.slots + 1 + offset)

    # ---------------------------------------------------------------- recall
    def ensure(self, indices, session, *, written=None, transient_start=None, keep_since=None,
               candidate_offset=0, gather_stream=None):
        """Exact recall of a logical selection; returns int32 physical pool ids.

        ``indices`` int32 ``[Q, K]`` on the pool device, ``-1`` padding. Ids
        below ``transient_start`` (or ``written``) are host-backed history;
        ids at or past ``transient_start`` are candidate rows. No host
        synchronisation unless the history exceeds the pool.

        Overlapped users (no reference counterpart): ``keep_since`` (the
        ``last_stamp`` of an earlier recall whose selection another stream
        still reads) keeps every slot that recall or a later one stamped out
        of the victims, and ``candidate_offset`` moves this call's candidate
        rows by that many rows (``write_candidates(..., offset=...)``). The
        pool contents then differ from the sequential FIFO order; every id
        still maps to a row holding its record. ``gather_stream`` (a
        ``torch.cuda.Stream``) takes the copy of the missing records, after
        the slot assignment on the current stream: readers of the records
        wait for it, and calls with a gather stream alternate between two
        workspaces, so a call may run while the previous call's copy does
        (the caller waits for the copy before the one after).
        """
        if indices.dtype != torch.int32 or indices.device != self.device:
            raise ValueError("indices must be int32 tensors on the pool device")
        self._check_live(session)
        written = session.written if written is None else written
        history = written if transient_start is None else transient_start
        if history > session.written:
            raise ValueError("host-backed history exceeds the session's written records")
        if type(candidate_offset) is not int or candidate_offset < 0:
            raise ValueError("candidate_offset must be a nonnegative integer")
        if keep_since is not None and (type(keep_since) is not int or not 0 <= keep_since < self.clock):
            raise ValueError("keep_since must be the stamp of an earlier recall")
        if transient_start is not None and not (
            0 <= written - transient_start <= self.candidate_slots - candidate_offset
        ):
            # cache/sparse_token_cache.py:254-256
            raise ValueError("transient suffix exceeds candidate slot capacity")
        union_checked = 0
        if history > self.slots:
            ids = indices[(indices >= 0) & (indices < history)]
            count = int(torch.unique(ids).numel())
            if count > self.slots:
                raise WorkingSetTooLarge(f"{count} selected history records exceed {self.slots} slots")
            union_checked = 1
        if self.clock + 2 >= MISSING:
            raise RuntimeError("FIFO clock exhausted")
        ids = indices.contiguous()
        physical = torch.empty_like(ids)
        protect, chosen = self.clock, self.clock + 1
        self.clock += 2
        self.last_stamp = protect
        pipelined = keep_since is not None or candidate_offset != 0 or gather_stream is not None
        workspace = self.workspace
        extra = ()
        if pipelined:
            gather = 0
            if gather_stream is not None:
                self.reserve_second_workspace()
                self._parity ^= 1
                workspace = self._second_workspace if self._parity else self.workspace
                gather = gather_stream.cuda_stream
            extra = (keep_since if keep_since is not None else -1, candidate_offset)
            tail = (_native.stream_of(self.device), gather)
        else:
            tail = (_native.stream_of(self.device),)
        with torch.cuda.device(self.device):
            _native.call(
                "dsa_pool_recall_pipelined" if pipelined else "dsa_pool_recall",
                _native.ptr(ids), ids.numel(), _native.ptr(session.page_table),
                history, written, -1 if transient_start is None else transient_start,
                self.slots, _native.ptr(self.host), self.host_capacity,
                _native.ptr(self.records), self.record_pages * PAGE_SIZE, RECORD_BYTES,
                _native.ptr(self.h2d), _native.ptr(self.d2h), _native.ptr(self.priority),
                protect, chosen, _native.ptr(workspace), workspace.numel(),
                self.history_capacity, union_checked, _native.ptr(self.stats),
                _native.ptr(self.status), _native.ptr(physical), *extra, *tail,
            )
        return physical

    def reserve_second_workspace(self):
        """Allocate the workspace that recalls with a gather stream alternate
        with (done once, outside any pipelined round)."""
        if self._second_workspace is None:
            self._second_workspace = torch.empty_like(self.workspace)

    def attend(self, q, physical, scale, value_dim=512, *, out=None):
        """Sparse MLA over recalled pool records (``sparse_mla_from_pool``);
        ``out`` (optional) receives the result."""
        rows = self.record_pages * PAGE_SIZE
        return attention.sparse_mla_fp8_paged(q, self.records, self.identity_pages, physical,
                                              scale, value_dim, n_tokens=rows, _out=out)

    def check_status(self):
        """Raise if a recall flagged an unwritten id or an overfull union (synchronises)."""
        value = int(self.status.item())
        self.status.zero_()
        if value & 4:
            raise ValueError("selection references unwritten cache records")
        if value & 8:
            raise WorkingSetTooLarge("a selection's union did not fit the pool")
        return value

    def metrics(self):
        union, recalled, evicted, _ = (int(x) for x in self.stats.tolist())
        return {
            "selection_records": union,
            "recalled_records": recalled,
            "evicted_records": evicted,
            "host_to_device_bytes": recalled * RECORD_BYTES,
        }
