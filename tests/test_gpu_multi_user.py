"""Overlapped multi-user layer step (``multi_user.MultiUserStep``) and the
pipelined recall it uses (``TokenPool.ensure(keep_since=..., candidate_offset=...)``)."""

import numpy as np
import pytest
import torch

from oracle import recall as orecall

pytestmark = pytest.mark.gpu


def _check_maps(pool):
    """The pool invariants of ``oracle.recall.check_maps`` on the device pool."""
    h2d = pool.h2d.cpu().numpy().astype(np.int64)
    d2h = pool.d2h.cpu().numpy()
    priority = pool.priority.cpu().numpy()
    live = np.nonzero(d2h != orecall.MISSING)[0]
    expected = pool.host[torch.from_numpy(d2h[live])].to(pool.device)
    got = pool.records.view(-1, 656)[torch.from_numpy(live).to(pool.device)]
    assert torch.equal(got, expected)
    assert d2h[0] == orecall.MISSING and priority[0] == orecall.MISSING
    assert np.array_equal(h2d[d2h[live]], live)
    host_live = np.nonzero(h2d != orecall.MISSING)[0]
    assert np.array_equal(d2h[h2d[host_live]], host_live)
    assert (priority[1:][d2h[1:] == orecall.MISSING] == -1).all()
    return len(live)


def test_keep_since_keeps_the_previous_selection(gpu):
    """When a recall needs more victims than the slots older than the kept
    selection, the keep floor turns the overflow into the short-pool status
    instead of evicting the kept slots; without the floor FIFO evicts them."""
    from cxldsagr_amd.token_pool import TokenPool, WorkingSetTooLarge

    gen = torch.Generator().manual_seed(3)
    order = torch.randperm(4096, generator=gen).int()
    old, held, new = order[:300], order[300:900], order[900:1400]
    kv = torch.randn(4096, 576, generator=gen).bfloat16().to(gpu)
    outcomes = []
    for floor in (True, False):
        pool = TokenPool(4096, 1000, device=gpu, candidate_slots=0)
        session = pool.allocate_session(4096)
        pool.write_history(session, kv)
        pool.ensure(old.view(1, -1).to(gpu), session)
        held_rows = pool.ensure(held.view(1, -1).to(gpu), session).clone()
        keep = pool.last_stamp
        pool.ensure(new.view(1, -1).to(gpu), session, keep_since=keep if floor else None)
        torch.cuda.synchronize()
        if floor:
            with pytest.raises(WorkingSetTooLarge):
                pool.check_status()
        else:
            assert pool.check_status() == 0
        h2d = pool.h2d.cpu()
        still = h2d[session.global_rows(0, 4096)[held.long()]]
        outcomes.append(bool(torch.equal(still, held_rows.view(-1).cpu())))
        _check_maps(pool)
    assert outcomes == [True, False]


def test_keep_since_and_candidate_offset_validation(gpu):
    from cxldsagr_amd.token_pool import TokenPool

    pool = TokenPool(128, 64, device=gpu, candidate_slots=8)
    session = pool.allocate_session(64)
    pool.write_history(session, torch.zeros(64, 576, dtype=torch.bfloat16, device=gpu))
    ids = torch.zeros(1, 4, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match="keep_since"):
        pool.ensure(ids, session, keep_since=0)  # no earlier recall yet
    pool.ensure(ids, session)
    with pytest.raises(ValueError, match="candidate_offset"):
        pool.ensure(ids, session, candidate_offset=-1)
    with pytest.raises(ValueError, match="candidate slot capacity"):
        pool.ensure(ids, session, written=68, transient_start=64, candidate_offset=6)


@pytest.mark.parametrize("users,history,rows,topk", [(5, 4096, 64, 512), (3, 8192, 128, 2048)])
def test_overlapped_users_equal_sequential_outputs(gpu, users, history, rows, topk):
    """Every user's output from the two-stream round equals, bit for bit,
    sparse MLA over a fully resident fp8 paged cache of the same records on the
    same selection, and the round's selections equal the sequential layer's."""
    from cxldsagr_amd.attention import pack_kv_fp8, sparse_mla_fp8_paged
    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.multi_user import MultiUserStep
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    tokens = history + rows
    slots = max(2 * history, users * history // 2)  # below the users' total: evictions happen
    pool = TokenPool(users * history, slots, device=gpu, candidate_slots=2 * rows,
                     history_capacity=history)
    pages = (tokens + 63) // 64
    identity = torch.arange(pages, dtype=torch.int32, device=gpu)
    layers, resident = [], []
    for u in range(users):
        inputs = make_layer_inputs(history, rows, seed=31 + u)
        layer = OffloadDSALayer(pool, pool.allocate_session(history), tokens, topk=topk)
        kv = inputs.kv[:history].to(gpu)
        layer.write_history(inputs.index_k[:history].to(gpu), kv)
        cache = torch.zeros(pages, 64, 656, dtype=torch.uint8, device=gpu)
        pack_kv_fp8(kv, cache, identity)
        layers.append(layer)
        resident.append(cache)
    step = MultiUserStep(layers)
    for rnd in range(2):
        batches = []
        for u in range(users):
            fresh = make_layer_inputs(0, rows, seed=1000 * (rnd + 1) + u)
            batches.append(tuple(getattr(fresh, n).to(gpu) for n in
                                 ("index_q", "index_k", "weights", "mla_q", "kv")))
        results = step.transient_round(batches)
        torch.cuda.synchronize()
        assert pool.check_status() == 0
        for u, (out, selection) in enumerate(results):
            layer, cache, b = layers[u], resident[u], batches[u]
            expected_ids = layer.select(b[0], b[1], b[2])
            assert torch.equal(selection.token_ids, expected_ids), (rnd, u)
            pack_kv_fp8(b[4], cache, identity, token_offset=history)
            expected = sparse_mla_fp8_paged(b[3], cache, identity, expected_ids, 576**-0.5,
                                            n_tokens=tokens)
            assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), (rnd, u)
        live = _check_maps(pool)
        assert 0 < live <= slots
    assert pool.metrics()["evicted_records"] > 0


@pytest.mark.parametrize("rows,chunks,commit", [(64, 2, False), (67, 3, False), (128, 4, True)])
def test_chunked_request_equals_resident_attention(gpu, rows, chunks, commit):
    """A request's batch in chunks of rows (``ChunkedForward``), each chunk's
    recall overlapping the next chunk's indexer: every output equals, bit for
    bit, sparse MLA over a fully resident fp8 cache of the same records on the
    same selection, and the selections equal ``select`` over the whole batch.
    Three users, two requests each, on a pool that holds two users' histories,
    so later requests evict; uneven chunks (67 rows in 3); transient and
    committed batches."""
    from cxldsagr_amd.attention import pack_kv_fp8, sparse_mla_fp8_paged
    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.multi_user import ChunkedForward
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    history, topk, users, visits = 4096, 2048, 3, 2
    grown = (history + visits * rows + 63) // 64 * 64   # whole 64-token host pages
    slots = 2 * grown
    pool = TokenPool(users * grown, slots, device=gpu, candidate_slots=rows,
                     history_capacity=grown)
    pipeline = ChunkedForward(pool, chunks)
    pages = (grown + 63) // 64
    identity = torch.arange(pages, dtype=torch.int32, device=gpu)
    layers, caches = [], []
    for u in range(users):
        inputs = make_layer_inputs(history, rows, seed=71 + u)
        layer = OffloadDSALayer(pool, pool.allocate_session(grown), grown + rows, topk=topk)
        kv = inputs.kv[:history].to(gpu)
        layer.write_history(inputs.index_k[:history].to(gpu), kv)
        cache = torch.zeros(pages, 64, 656, dtype=torch.uint8, device=gpu)
        pack_kv_fp8(kv, cache, identity)
        layers.append(layer)
        caches.append(cache)
    for visit in range(visits):
        for u in range(users):
            layer, cache = layers[u], caches[u]
            fresh = make_layer_inputs(0, rows, seed=5000 + 100 * visit + u)
            index_q, index_k, weights, q, kv = (getattr(fresh, n).to(gpu) for n in
                                                ("index_q", "index_k", "weights", "mla_q", "kv"))
            position = layer.written
            assert pipeline.overlaps(layer, rows, transient=not commit)
            print(f"chunked request: user {u} visit {visit} rows {rows} chunks {chunks}", flush=True)
            out, selection = pipeline.forward(layer, index_q, index_k, weights, q, kv,
                                              transient=not commit)
            torch.cuda.synchronize()
            assert pool.check_status() == 0
            assert layer.written == position + (rows if commit else 0)
            expected_ids = layer.select(index_q, index_k, weights, position=position)
            assert torch.equal(selection.token_ids, expected_ids), (visit, u)
            pack_kv_fp8(kv, cache, identity, token_offset=position)
            expected = sparse_mla_fp8_paged(q, cache, identity, expected_ids, 576**-0.5,
                                            n_tokens=position + rows)
            assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), (visit, u)
        live = _check_maps(pool)
        assert 0 < live <= slots
    assert pool.metrics()["evicted_records"] > 0


def test_chunked_request_runs_sequentially_when_two_chunks_may_not_fit(gpu):
    """With less than two histories of slots the pipeline would have to evict
    the previous chunk's kept slots: it runs the batch as ``forward`` does."""
    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.multi_user import ChunkedForward
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    history, rows = 4096, 64
    pool = TokenPool(history, history + 100, device=gpu, candidate_slots=rows,
                     history_capacity=history)
    inputs = make_layer_inputs(history, rows, seed=9)
    layer = OffloadDSALayer(pool, pool.allocate_session(history), history + rows, topk=2048)
    layer.write_history(inputs.index_k[:history].to(gpu), inputs.kv[:history].to(gpu))
    pipeline = ChunkedForward(pool, 2)
    assert not pipeline.overlaps(layer, rows, transient=True)
    batch = [getattr(inputs, n)[-rows:].to(gpu) if n in ("index_k", "kv") else getattr(inputs, n).to(gpu)
             for n in ("index_q", "index_k", "weights", "mla_q", "kv")]
    out, selection = pipeline.forward(layer, *batch, transient=True)
    again, second = layer.forward(*batch, transient=True)
    torch.cuda.synchronize()
    assert torch.equal(selection.token_ids, second.token_ids)
    assert torch.equal(out.view(torch.int16), again.view(torch.int16))
    with pytest.raises(ValueError, match="chunks"):
        ChunkedForward(pool, 0)
