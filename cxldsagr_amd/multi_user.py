"""Several sessions' layer steps over one shared token pool, the recall of one
user overlapping the indexer and sparse MLA of its neighbours.

The reference's multi-user GR runner steps its users one after another per
layer (``serving/persistent.py:56``; per user ``_consume`` of
``models/deepseek_v32/attention.py:201-235``: recall, then sparse MLA), so
every user's PCIe recall is exposed. Here one layer of a round of users runs
as a three-stream pipeline on the pool's device:

* compute stream: user u's indexer (quantise, logits, top-k) and candidate
  write, then user u - 1's sparse MLA over the pool;
* recall stream: user u's recall bookkeeping (union, victims, maps), after
  user u's top-k and after user u - 2's copy (whose workspace it reuses);
* copy stream: user u's copy of the missing records over PCIe, after user
  u's bookkeeping and after user u - 1's sparse MLA. The copy kernel keeps
  waves resident on every CU while the link drains, and the sparse MLA
  kernel needs each SIMD's whole register file per wave, so the two would
  not run side by side anyway: the copies and the MLAs alternate, and the
  indexer and the recall bookkeeping of the next user hide under each copy.

User u's recall keeps user u - 1's slots out of its victims (``keep_since``)
while that user's MLA may still be reading them, and users alternate between
two halves of the candidate rows, so no row is overwritten before its reader
is done. Every selected id still resolves to a row holding its record, so each
user's output equals, bit for bit, the sequential step's; only the pool's
victim choice (which slots hold what) differs from the sequential FIFO order.
"""

import torch

from cxldsagr_amd.layer import OffloadDSALayer, TokenSelection


class MultiUserStep:
    """One layer for a list of ``OffloadDSALayer`` s that share one ``TokenPool``.

    The pool needs candidate rows for two batches in flight
    (``candidate_slots >= 2 * rows``) and room for two users' selections at
    once (``2 * history <= slots`` for every session, so that a recall never
    runs out of victims while the previous user's slots are kept).
    """

    def __init__(self, layers):
        if not layers or not all(isinstance(layer, OffloadDSALayer) for layer in layers):
            raise ValueError("MultiUserStep needs a nonempty list of OffloadDSALayer")
        pool = layers[0].pool
        if any(layer.pool is not pool for layer in layers):
            raise ValueError("all sessions must share one token pool")
        self.layers, self.pool, self.device = list(layers), pool, pool.device
        self._recall_stream = torch.cuda.Stream(self.device)
        self._copy_stream = torch.cuda.Stream(self.device)
        pool.reserve_second_workspace()

    def transient_round(self, batches):
        """GR candidate step for every user: ``batches[u]`` is
        ``(index_q, index_k, weights, q, kv)`` of user u's candidate tokens at
        its ``session.written``. Returns ``[(out, TokenSelection), ...]`` in
        user order, enqueued on the current stream (no host synchronisation)."""
        if len(batches) != len(self.layers):
            raise ValueError("one batch per user")
        pool = self.pool
        rows = {len(b[0]) for b in batches}
        if len(rows) != 1:
            raise ValueError("every user's batch must have the same number of rows")
        rows = rows.pop()
        if 2 * rows > pool.candidate_slots:
            raise ValueError("overlapped users need candidate rows for two batches")
        for layer, batch in zip(self.layers, batches):
            if 2 * layer.session.written > pool.slots:
                raise ValueError("overlapped recall needs room for two users' selections")
            if any(len(x) != rows for x in batch):
                raise ValueError("query batch inputs disagree in length")
        compute = torch.cuda.current_stream(self.device)
        recall, copy = self._recall_stream, self._copy_stream
        n = len(self.layers)
        selected, recalled, copied, done = ([torch.cuda.Event() for _ in range(n)] for _ in range(4))
        ids, physical, outs = [None] * n, [None] * n, [None] * n
        keep = None
        for u in range(n + 1):
            if u < n:
                layer = self.layers[u]
                index_q, index_k, weights, q, kv = batches[u]
                position = layer.session.written
                offset = (u % 2) * rows
                ids[u] = layer.select(index_q, index_k, weights)
                pool.write_candidates(kv, offset=offset)
                selected[u].record(compute)
                recall.wait_event(selected[u])
                if u >= 2:
                    recall.wait_event(copied[u - 2])
                if u >= 1:
                    copy.wait_event(done[u - 1])
                with torch.cuda.stream(recall):
                    physical[u] = pool.ensure(ids[u], layer.session, written=position + rows,
                                              transient_start=position, keep_since=keep,
                                              candidate_offset=offset, gather_stream=copy)
                keep = pool.last_stamp
                ids[u].record_stream(recall)
                recalled[u].record(recall)
                copied[u].record(copy)
            if u >= 1:
                v = u - 1
                compute.wait_event(recalled[v])
                compute.wait_event(copied[v])
                physical[v].record_stream(compute)
                outs[v] = pool.attend(batches[v][3], physical[v], self.layers[v].scale)
                done[v].record(compute)
        return [(outs[u], TokenSelection(ids[u])) for u in range(n)]


class ChunkedForward:
    """One session's query batch as a pipeline of row chunks, within one
    request: chunk c's recall overlaps chunk c + 1's indexer and chunk c - 1's
    sparse MLA.

    The reference overlaps a request's host-to-HBM traffic with its own
    indexer by prefetching, from inside the fused logits kernel, the tokens
    that a histogram of earlier query rows' scores proves to be in their
    top-2048 (``indexer/csrc/echo_logits.cuh:527-584``), and recalls the rest
    exactly afterwards. Here each chunk's exact selection is recalled as soon
    as its top-k is known, on the three streams ``MultiUserStep`` uses:

    * compute stream: chunk c's indexer (prologue, logits, top-k over its rows
      at their own causal positions), then chunk c - 1's sparse MLA into its
      rows of the output;
    * recall stream: chunk c's recall bookkeeping, after chunk c's top-k and
      after chunk c - 2's copy (whose workspace it reuses);
    * copy stream: chunk c's copy of its missing records, after its
      bookkeeping and after chunk c - 1's sparse MLA.

    Chunk c's recall keeps chunk c - 1's slots out of its victims while that
    chunk's MLA may still read them, so the pool must hold two chunks'
    selections at once: ``2 * history <= pool.slots``. When it does not (or
    with one chunk) the batch runs as ``OffloadDSALayer.forward`` does.
    Outputs and selections equal ``OffloadDSALayer.forward``'s bit for bit;
    only the pool's victim choice differs from the sequential FIFO order.
    """

    def __init__(self, pool, chunks=2):
        if type(chunks) is not int or chunks < 1:
            raise ValueError("chunks must be a positive integer")
        self.pool, self.chunks, self.device = pool, chunks, pool.device
        self._recall_stream = torch.cuda.Stream(self.device)
        self._copy_stream = torch.cuda.Stream(self.device)
        pool.reserve_second_workspace()

    def overlaps(self, layer, rows, *, transient):
        """Whether ``forward`` pipelines this batch (else it runs sequentially)."""
        history = layer.session.written + (0 if transient else rows)
        return self.chunks > 1 and rows > 1 and 2 * history <= self.pool.slots

    def forward(self, layer, index_q, index_k, weights, q, kv, *, transient=False):
        """``layer.forward(index_q, index_k, weights, q, kv, transient=...)``
        with the recall of each chunk of rows overlapped; enqueued on the
        current stream, returns ``(out, TokenSelection)``."""
        if not isinstance(layer, OffloadDSALayer) or layer.pool is not self.pool:
            raise ValueError("the layer must use this pipeline's token pool")
        rows = len(index_q)
        if not self.overlaps(layer, rows, transient=transient):
            return layer.forward(index_q, index_k, weights, q, kv, transient=transient)
        pool, session = self.pool, layer.session
        position = session.written
        end = position + rows
        if end > layer.capacity or any(len(x) != rows for x in (index_k, weights, q, kv)):
            raise ValueError("query batch exceeds the layer capacity or inputs disagree in length")
        if transient and rows > pool.candidate_slots:
            raise ValueError("transient suffix exceeds candidate slot capacity")
        # Every chunk's records first: a chunk's rows see the earlier rows of the batch.
        if transient:
            pool.write_candidates(kv)
            transient_start = position
        else:
            pool.append_records(session, kv)
            transient_start = None
        chunks = min(self.chunks, rows)
        bounds = [rows * c // chunks for c in range(chunks + 1)]
        compute = torch.cuda.current_stream(self.device)
        recall, copy = self._recall_stream, self._copy_stream
        selected, recalled, copied, done = ([torch.cuda.Event() for _ in range(chunks)]
                                            for _ in range(4))
        ids = torch.empty((rows, layer.topk), dtype=torch.int32, device=self.device)
        out = torch.empty((rows, q.shape[1], 512), dtype=q.dtype, device=self.device)
        physical = [None] * chunks
        keep = None
        for c in range(chunks + 1):
            if c < chunks:
                lo, hi = bounds[c], bounds[c + 1]
                ids[lo:hi] = layer.select(index_q[lo:hi], index_k[lo:hi], weights[lo:hi],
                                          position=position + lo)
                selected[c].record(compute)
                recall.wait_event(selected[c])
                if c >= 2:
                    recall.wait_event(copied[c - 2])
                if c >= 1:
                    copy.wait_event(done[c - 1])
                with torch.cuda.stream(recall):
                    physical[c] = pool.ensure(ids[lo:hi], session, written=end,
                                              transient_start=transient_start, keep_since=keep,
                                              gather_stream=copy)
                keep = pool.last_stamp
                recalled[c].record(recall)
                copied[c].record(copy)
            if c >= 1:
                v = c - 1
                lo, hi = bounds[v], bounds[v + 1]
                compute.wait_event(recalled[v])
                compute.wait_event(copied[v])
                physical[v].record_stream(compute)
                pool.attend(q[lo:hi], physical[v], layer.scale, out=out[lo:hi])
                done[v].record(compute)
        ids.record_stream(recall)
        return out, TokenSelection(ids)
