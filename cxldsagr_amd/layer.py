"""One DSA prefill layer on MI355X: indexer -> exact top-k -> sparse MLA.

Follows the stage order of the reference's ``EchoAttentionRunner._forward``
(``models/deepseek_v32/attention.py:276-425``) for the hot path:

1. quantise the indexer Q (A1) and fold ``q_scale`` into the head weights
   in the same kernel (``models/deepseek_v32/projections.py:241-244``; A2);
2. quantise the new tokens' index K straight into the resident index cache
   (``attention.py:323-326``; A3);
3. fp8 logits with the causal ``-inf`` tail (``attention.py:338-353``; A4),
   written only as top-k candidates: the scores at or above a per-row floor
   estimated from a sample of the row;
4. exact top-k of those candidates (``attention.py:358-370``; A6), fused
   with step 3 through ``indexer.select_topk`` (no score matrix);
5. append the new tokens' KV records (quantise-on-append into the fp8 paged
   cache, or a bf16 copy) (``attention.py:400-401``);
6. sparse MLA over the selection (``attention.py:201-235``; A7).

Projections and the output projection stay outside this layer (the
reference's ``project``/``output`` callbacks). All stages run on the current
stream without host synchronisation.
"""

import torch

from cxldsagr_amd import _native, attention, indexer
from cxldsagr_amd.contracts import AttentionContext, TokenSelection

PAGE_TOKENS = 64


def index_prologue_applies(index_q, index_k, weights, device):
    """The one-launch prologue covers the model shapes (bf16 index Q
    ``[rows, 64, 128]`` and K ``[rows, 128]``, f32 weights ``[rows, 64]``)."""
    rows = len(index_q)
    return (index_q.dtype == torch.bfloat16 and index_q.ndim == 3
            and index_q.shape[1:] == (64, 128) and index_k.dtype == torch.bfloat16
            and tuple(index_k.shape) == (rows, 128) and weights.dtype == torch.float32
            and tuple(weights.shape) == (rows, 64)
            and all(t.device == device for t in (index_q, index_k, weights)))


def index_prologue(index_q, index_k, weights, index_keys, index_scales, position, topk, floors,
                   *, kv=None, page_table=None, kv_cache=None):
    """The small stages before the indexer's logits in one launch
    (``dsa_layer_prologue_floors_fp8``): Q quantisation + weight fold, the new
    index K quantised into the resident cache at ``position``, the new KV
    records packed into the fp8 paged cache (when ``kv`` is given), and, with
    ``floors`` (int32 ``[rows, 2]``), the candidate top-k's per-row floors -
    the same bits as the separate operators. Returns ``(q8, folded, q_fold)``,
    ``q_fold`` the partial folded queries ``[rows, 4, 128]`` that let the
    logits kernel skip forming them (same logits bits)."""
    device = index_q.device
    rows = len(index_q)
    end = position + rows
    index_q, index_k, weights = (t.contiguous() for t in (index_q, index_k, weights))
    index_q, index_k = (attention._aligned(t) for t in (index_q, index_k))
    q8 = torch.empty(index_q.shape, dtype=torch.float8_e4m3fn, device=device)
    q_scales = torch.empty((*index_q.shape[:-1], 1), dtype=torch.float32, device=device)
    folded = torch.empty_like(weights)
    q_fold = torch.empty((rows, 4, 128), dtype=torch.float32, device=device)
    if kv is not None:
        kv = attention._aligned(kv.contiguous())
    with torch.cuda.device(device):
        _native.call(
            "dsa_layer_prologue_floors_fp8",
            _native.ptr(index_q), rows * 64, _native.ptr(weights), _native.ptr(q8),
            _native.ptr(q_scales), _native.ptr(folded), _native.ptr(q_fold),
            _native.ptr(index_k), rows, _native.ptr(index_keys[position:end]),
            _native.ptr(index_scales[position:end]),
            _native.ptr(kv), rows if kv is not None else 0, position if kv is not None else 0,
            _native.ptr(page_table),
            kv_cache.shape[0] if kv is not None else 0, _native.ptr(kv_cache), None,
            _native.ptr(index_keys), _native.ptr(index_scales), position, topk,
            _native.ptr(floors), _native.stream_of(device),
        )
    return q8, folded, q_fold


class DSALayer:
    """Resident HBM caches for one layer of one sequence.

    ``kv_format`` is ``"fp8_paged"`` (656-byte records in 64-token pages behind
    ``page_table``) or ``"bf16"`` (flat 1152-byte records, the reference's
    format). Implements the ``CacheAccess`` protocol for its own sequence.
    """

    def __init__(self, capacity, *, device, heads=128, topk=2048, scale=576**-0.5,
                 kv_format="fp8_paged", page_table=None, pages=None, layer_idx=0):
        if kv_format not in ("fp8_paged", "bf16"):
            raise ValueError("kv_format must be 'fp8_paged' or 'bf16'")
        if type(capacity) is not int or capacity < 1:
            raise ValueError("capacity must be a positive integer")
        self.device = torch.device(device)
        self.capacity, self.heads, self.topk, self.scale = capacity, heads, topk, scale
        self.kv_format, self.layer_idx = kv_format, layer_idx
        self.index_keys = torch.zeros((capacity, 128), dtype=torch.float8_e4m3fn, device=self.device)
        self.index_scales = torch.zeros(capacity, dtype=torch.float32, device=self.device)
        logical_pages = (capacity + PAGE_TOKENS - 1) // PAGE_TOKENS
        if kv_format == "fp8_paged":
            if page_table is None:
                page_table = torch.arange(logical_pages, dtype=torch.int32)
            self.page_table = page_table.to(device=self.device, dtype=torch.int32).contiguous()
            if self.page_table.numel() < logical_pages:
                raise ValueError("page_table must cover the layer capacity")
            pages = logical_pages if pages is None else pages
            self.kv_cache = torch.zeros((pages, PAGE_TOKENS, attention.RECORD_BYTES),
                                        dtype=torch.uint8, device=self.device)
            self.records = None
        else:
            self.page_table = None
            self.kv_cache = None
            self.records = torch.zeros((capacity, attention.QK_DIM), dtype=torch.bfloat16,
                                       device=self.device)
        self.written = 0
        self._state = {}

    # ------------------------------------------------------------ CacheAccess
    @property
    def length(self):
        return self.written

    @property
    def max_seq_len(self):
        return self.capacity

    def get_layer_state(self, layer_idx):
        return self._state.get(layer_idx)

    def set_layer_state(self, layer_idx, state):
        self._state[layer_idx] = state

    # ---------------------------------------------------------------- writes
    def _append_kv(self, kv, start):
        if self.kv_format == "fp8_paged":
            attention.pack_kv_fp8(kv, self.kv_cache, self.page_table, token_offset=start)
        else:
            self.records[start:start + len(kv)].copy_(kv)

    def write_history(self, index_k, kv):
        """Bulk-append already projected history tokens (bf16 index K and KV)."""
        start, end = self.written, self.written + len(index_k)
        if len(kv) != len(index_k) or end > self.capacity:
            raise ValueError("history exceeds the layer capacity or K/KV lengths differ")
        indexer.quantize_into(index_k, self.index_keys[start:end], self.index_scales[start:end])
        self._append_kv(kv, start)
        self.written = end
        return start

    # ---------------------------------------------------------------- stages
    def index(self, index_q, index_k, weights, position):
        """Indexer: A1 -> A2 -> A3 -> A4 -> A6. Returns the TokenSelection."""
        rows = len(index_q)
        end = position + rows
        if end > self.capacity:
            raise ValueError("query batch exceeds the layer capacity")
        if index_prologue_applies(index_q, index_k, weights, self.device):
            floors = indexer.select_floors_buffer(self.device, rows, end)
            q8, folded, q_fold = index_prologue(index_q, index_k, weights, self.index_keys,
                                                self.index_scales, position, self.topk, floors)
            _, ids = indexer.select_topk(q8, self.index_keys[:end], folded,
                                         self.index_scales[:end], position, self.topk,
                                         _q_fold=q_fold, _floors_ready=True)
            return TokenSelection(ids)
        q8, _, weights = indexer.quantize_index_folded(index_q, weights)
        indexer.quantize_into(index_k, self.index_keys[position:end],
                              self.index_scales[position:end])
        _, ids = indexer.select_topk(q8, self.index_keys[:end], weights,
                                     self.index_scales[:end], position, self.topk)
        return TokenSelection(ids)

    def consume(self, q, selection, kv, position):
        """Main attention: append the new KV, then sparse MLA over the selection."""
        end = position + len(q)
        self._append_kv(kv, position)
        return self._attend(q, selection.token_ids, end)

    def _fused_prologue_applies(self, index_q, index_k, weights, kv):
        """The one-launch prologue covers the model shapes on the fp8 paged cache."""
        rows = len(index_q)
        return (self.kv_format == "fp8_paged" and index_q.dtype == torch.bfloat16
                and index_q.ndim == 3 and index_q.shape[1:] == (64, 128)
                and index_k.dtype == torch.bfloat16 and tuple(index_k.shape) == (rows, 128)
                and weights.dtype == torch.float32 and tuple(weights.shape) == (rows, 64)
                and kv.dtype == torch.bfloat16 and tuple(kv.shape) == (rows, attention.QK_DIM)
                and all(t.device == self.device for t in (index_q, index_k, weights, kv)))

    def _prologue(self, index_q, index_k, weights, kv, position, floors=None):
        """Q quantisation + weight fold, new index K into the cache and the new
        KV records into the fp8 paged cache, in one launch (``index_prologue``).
        Returns ``(q8, folded, q_fold)``."""
        return index_prologue(index_q, index_k, weights, self.index_keys, self.index_scales,
                              position, self.topk, floors, kv=kv, page_table=self.page_table,
                              kv_cache=self.kv_cache)

    def _attend(self, q, ids, end):
        if self.kv_format == "fp8_paged":
            return attention.sparse_mla_fp8_paged(q, self.kv_cache, self.page_table, ids,
                                                  self.scale, n_tokens=end)
        return attention.sparse_mla(q, self.records[:end], ids, self.scale)

    def forward(self, index_q, index_k, weights, q, kv):
        """Run one query batch at ``position = self.written``; returns (out, selection).

        The stages of ``index`` then ``consume`` in one call (the KV append
        placed after the top-k, where the runner's ``consume`` does it).
        """
        position = self.written
        rows = len(index_q)
        end = position + rows
        if end > self.capacity or len(q) != rows or len(kv) != rows or len(index_k) != rows:
            raise ValueError("query batch exceeds the layer capacity or inputs disagree in length")
        q_fold = floors = None
        if self._fused_prologue_applies(index_q, index_k, weights, kv):
            floors = indexer.select_floors_buffer(self.device, rows, end)
            q8, folded, q_fold = self._prologue(index_q, index_k, weights, kv, position, floors)
        elif index_prologue_applies(index_q, index_k, weights, self.device):
            floors = indexer.select_floors_buffer(self.device, rows, end)
            q8, folded, q_fold = index_prologue(index_q, index_k, weights, self.index_keys,
                                                self.index_scales, position, self.topk, floors)
            self._append_kv(kv, position)
        else:
            indexer.quantize_into(index_k, self.index_keys[position:end],
                                  self.index_scales[position:end])
            q8, _, folded = indexer.quantize_index_folded(index_q, weights)
            self._append_kv(kv, position)
        _, ids = indexer.select_topk(q8, self.index_keys[:end], folded,
                                     self.index_scales[:end], position, self.topk,
                                     _q_fold=q_fold, _floors_ready=floors is not None)
        selection = TokenSelection(ids)
        out = self._attend(q, ids, end)
        self.written = end
        return out, selection

    def forward_projected(self, projection, projected, q, kv):
        """``forward`` from the indexer's GEMM outputs (``projections.IndexProjected``).

        One producer launch (``projections.index_producer``: K LayerNorm,
        both RoPEs, both quantisations, the weight fold, the index-cache write
        and, for the fp8 paged cache, the new KV records) takes the place of
        the prologue; then the fused logits/top-k and sparse MLA as in
        ``forward``. ``projection`` is the layer's ``IndexerProjection``.
        """
        position = self.written
        rows = len(q)
        end = position + rows
        if (end > self.capacity or len(kv) != rows or projected.q_proj.shape[0] != rows
                or projected.k_proj.shape[0] != rows):
            raise ValueError("query batch exceeds the layer capacity or inputs disagree in length")
        paged = self.kv_format == "fp8_paged"
        floors = indexer.select_floors_buffer(self.device, rows, end)
        q8, _, folded, _, _, q_fold = projection.produce(
            projected, index_keys=self.index_keys[position:end],
            index_scales=self.index_scales[position:end], q_fold=True,
            kv=kv if paged else None, kv_cache=self.kv_cache, page_table=self.page_table,
            token_offset=position, floors=floors, key_cache=self.index_keys,
            key_cache_scales=self.index_scales, topk=self.topk)
        if not paged:
            self._append_kv(kv, position)
        _, ids = indexer.select_topk(q8, self.index_keys[:end], folded,
                                     self.index_scales[:end], position, self.topk,
                                     _q_fold=q_fold, _floors_ready=True)
        out = self._attend(q, ids, end)
        self.written = end
        return out, TokenSelection(ids)


class OffloadDSALayer:
    """One layer of one session whose KV records live in a bounded HBM token pool.

    The offload half of the reference runner (``attention.py:201-235``): the
    indexer keys stay resident (as in the reference); the main KV records sit
    in the pool's pinned host arena and only the selected ones are recalled
    into the pool's slots before sparse MLA reads them by physical id. New
    tokens are either persistent (written to the session's host pages, then
    recalled like history when selected) or transient GR candidates (written
    to the pool's candidate rows and never committed,
    ``cache/sparse_token_cache.py:244-318``).

    ``consume`` mirrors ``_consume``: exact recall of the selection; when its
    union does not fit the pool (``WorkingSetTooLarge``), the query batch is
    halved recursively and the halves concatenated, and a single query whose
    selection does not fit raises ``ValueError``. ``capacity_splits`` counts
    the splits as the reference's ``stats.capacity_splits`` does.
    """

    def __init__(self, pool, session, capacity, *, topk=2048, scale=576**-0.5, layer_idx=0):
        # The index-K capacity may exceed the session's host pages: transient
        # candidate tokens have index keys but no host records.
        if type(capacity) is not int or capacity < 1:
            raise ValueError("capacity must be a positive integer")
        self.pool, self.session = pool, session
        self.device = pool.device
        self.capacity, self.topk, self.scale, self.layer_idx = capacity, topk, scale, layer_idx
        self.index_keys = torch.zeros((capacity, 128), dtype=torch.float8_e4m3fn, device=self.device)
        self.index_scales = torch.zeros(capacity, dtype=torch.float32, device=self.device)
        self.capacity_splits = 0

    @property
    def written(self):
        return self.session.written

    def write_history(self, index_k, kv):
        """Bulk-append projected history: index K into the resident cache, KV records
        (fp8-packed) into the session's host pages."""
        start, end = self.session.written, self.session.written + len(index_k)
        if len(kv) != len(index_k) or end > self.capacity:
            raise ValueError("history exceeds the layer capacity or K/KV lengths differ")
        indexer.quantize_into(index_k, self.index_keys[start:end], self.index_scales[start:end])
        self.pool.write_history(self.session, kv)
        return start

    def forward(self, index_q, index_k, weights, q, kv, *, transient=False):
        """One query batch at ``position = session.written``; returns (out, selection).

        ``transient=True`` runs the GR candidate step: the batch's KV goes to
        the pool's candidate rows and the session's history is not extended.
        """
        position = self.session.written
        rows = len(index_q)
        end = position + rows
        if end > self.capacity or len(q) != rows or len(kv) != rows or len(index_k) != rows:
            raise ValueError("query batch exceeds the layer capacity or inputs disagree in length")
        if transient and rows > self.pool.candidate_slots:
            raise ValueError("transient suffix exceeds candidate slot capacity")
        ids = self.select(index_q, index_k, weights)
        if transient:
            self.pool.write_candidates(kv)
            out = self.consume(q, ids, written=end, transient_start=position)
        else:
            self.pool.append_records(self.session, kv)
            out = self.consume(q, ids, written=end)
        return out, TokenSelection(ids)

    def select(self, index_q, index_k, weights, *, position=None):
        """The indexer half of ``forward`` for a batch at ``position`` (default
        ``session.written``): quantise the batch's index Q (folding its scales
        into the head weights) and index K (into the resident cache), fp8
        logits over every visible key, exact top-k; returns the int32
        ``[rows, topk]`` ids. Keys before ``position`` must be in the cache."""
        position = self.session.written if position is None else position
        if type(position) is not int or position < 0:
            raise ValueError("position must be a nonnegative integer")
        end = position + len(index_q)
        if end > self.capacity or len(index_k) != len(index_q) or len(weights) != len(index_q):
            raise ValueError("query batch exceeds the layer capacity or inputs disagree in length")
        rows = len(index_q)
        if index_prologue_applies(index_q, index_k, weights, self.device):
            # Quantisers and the candidate top-k's floors in one launch.
            floors = indexer.select_floors_buffer(self.device, rows, end)
            q8, folded, q_fold = index_prologue(index_q, index_k, weights, self.index_keys,
                                                self.index_scales, position, self.topk, floors)
            _, ids = indexer.select_topk(q8, self.index_keys[:end], folded,
                                         self.index_scales[:end], position, self.topk,
                                         _q_fold=q_fold, _floors_ready=True)
            return ids
        q8, _, folded = indexer.quantize_index_folded(index_q, weights)
        indexer.quantize_into(index_k, self.index_keys[position:end], self.index_scales[position:end])
        _, ids = indexer.select_topk(q8, self.index_keys[:end], folded,
                                     self.index_scales[:end], position, self.topk)
        return ids

    def consume(self, q, ids, *, written, transient_start=None):
        """Recall then sparse MLA over the pool, splitting the query batch on
        ``WorkingSetTooLarge`` (``attention.py:213-228``)."""
        from cxldsagr_amd.token_pool import WorkingSetTooLarge

        try:
            physical = self.pool.ensure(ids, self.session, written=written,
                                        transient_start=transient_start)
        except WorkingSetTooLarge:
            if len(q) == 1:
                raise ValueError("offload slots must fit at least one query's exact selection") from None
            self.capacity_splits += 1
            middle = len(q) // 2
            left = self.consume(q[:middle], ids[:middle], written=written,
                                transient_start=transient_start)
            right = self.consume(q[middle:], ids[middle:], written=written,
                                 transient_start=transient_start)
            return torch.cat((left, right))
        return self.pool.attend(q, physical, self.scale)


class LayerIndexer:
    """``Indexer`` protocol adapter: ``context.auxiliary_state`` carries the new
    tokens' bf16 index K (``"index_k"``) and head weights (``"weights"``)."""

    def __init__(self, layer):
        self.layer = layer

    def __call__(self, q, cache_access, context: AttentionContext):
        aux = context.auxiliary_state
        return self.layer.index(q, aux["index_k"], aux["weights"], context.query_start)


class LayerAttention:
    """``MainAttention`` protocol adapter: ``context.auxiliary_state["kv"]`` holds
    the new tokens' bf16 KV records."""

    def __init__(self, layer):
        self.layer = layer

    def __call__(self, q, selection, cache_access, context: AttentionContext):
        if not isinstance(selection, TokenSelection):
            raise ValueError("DSA main attention consumes a TokenSelection")
        out = self.layer.consume(q, selection, context.auxiliary_state["kv"], context.query_start)
        self.layer.written = max(self.layer.written, context.query_start + len(q))
        return out
