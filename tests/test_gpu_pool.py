"""GPU exact recall (A10) state-for-state against the oracle, and MLA over the pool."""

import numpy as np
import pytest
import torch

from oracle import recall as orecall

pytestmark = pytest.mark.gpu


def _state(pool):
    return {
        "h2d": pool.h2d.cpu().numpy().astype(np.int64),
        "d2h": pool.d2h.cpu().numpy(),
        "priority": pool.priority.cpu().numpy(),
        "records": pool.records.view(-1, 656)[: pool.slots + 1 + pool.candidate_slots].cpu().numpy(),
    }


def _mirror(pool):
    mirror = orecall.Pool(pool.host_capacity, pool.slots, 656, pool.candidate_slots)
    mirror.host[:] = pool.host.numpy()
    return mirror


@pytest.mark.parametrize("seed,slots", [(0, 300), (1, 300), (2, 1000), (3, 64)])
def test_recall_sequences_match_oracle_state(gpu, seed, slots):
    from cxldsagr_amd.token_pool import TokenPool

    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    pool = TokenPool(1024, slots, device=gpu, candidate_slots=16, history_capacity=1024)
    session = pool.allocate_session(1024)
    tokens = 900
    pool.write_history(session, torch.randn(tokens, 576, generator=gen).bfloat16().to(gpu))
    mirror = _mirror(pool)
    table = session.page_table.cpu().numpy()
    for step in range(10):
        q = int(rng.integers(1, 5))
        k = int(rng.integers(1, max(2, slots // 4)))  # q * k <= slots: the union fits
        limit = tokens
        sel = rng.integers(-2, limit, (q, k)).astype(np.int32)
        if slots < 100:
            # keep each union within the pool
            base = rng.integers(0, limit - 40)
            sel = (base + rng.integers(0, 40, (q, k))).astype(np.int32)
            sel[rng.random((q, k)) < 0.1] = -1
        expected = orecall.ensure(mirror, sel, table, written=tokens)
        physical = pool.ensure(torch.from_numpy(sel).to(gpu), session, written=tokens)
        torch.cuda.synchronize()
        assert pool.check_status() == 0
        np.testing.assert_array_equal(physical.cpu().numpy(), expected)
        state = _state(pool)
        np.testing.assert_array_equal(state["h2d"], mirror.h2d)
        np.testing.assert_array_equal(state["d2h"], mirror.d2h)
        np.testing.assert_array_equal(state["priority"], mirror.priority)
        np.testing.assert_array_equal(state["records"], mirror.records)
    metrics = pool.metrics()
    assert metrics["recalled_records"] == mirror.recalled
    assert metrics["evicted_records"] == mirror.evicted


def test_transient_candidates_and_pool_attention_equal_resident_attention(gpu):
    from cxldsagr_amd.attention import pack_kv_fp8, sparse_mla_fp8_paged
    from cxldsagr_amd.token_pool import TokenPool

    gen = torch.Generator().manual_seed(9)
    history, cands = 3000, 32
    kv = torch.randn(history + cands, 576, generator=gen).bfloat16().to(gpu)
    pool = TokenPool(4096, 1024, device=gpu, candidate_slots=64)
    session = pool.allocate_session(4096)
    pool.write_history(session, kv[:history])
    pool.write_candidates(kv[history:])
    # resident reference: the same tokens in a fully resident fp8 paged cache
    pages = (history + cands + 63) // 64
    cache = torch.zeros(pages, 64, 656, dtype=torch.uint8, device=gpu)
    table = torch.arange(pages, dtype=torch.int32, device=gpu)
    pack_kv_fp8(kv, cache, table)
    q = torch.randn(8, 128, 576, generator=gen).bfloat16().to(gpu)
    sel = torch.randint(-1, history + cands, (8, 96), generator=gen).int().to(gpu)
    physical = pool.ensure(sel, session, written=history + cands, transient_start=history)
    out_pool = pool.attend(q, physical, 576**-0.5)
    out_resident = sparse_mla_fp8_paged(q, cache, table, sel, 576**-0.5, n_tokens=history + cands)
    assert pool.check_status() == 0
    assert torch.equal(out_pool.view(torch.int16), out_resident.view(torch.int16))
    cand = sel >= history
    assert torch.equal(physical[cand], (sel[cand] - history + pool.slots + 1).int())


def test_oversize_union_raises_before_launch(gpu):
    from cxldsagr_amd.token_pool import TokenPool, WorkingSetTooLarge

    gen = torch.Generator().manual_seed(4)
    pool = TokenPool(512, 64, device=gpu)
    session = pool.allocate_session(512)
    pool.write_history(session, torch.randn(500, 576, generator=gen).bfloat16().to(gpu))
    with pytest.raises(WorkingSetTooLarge):
        pool.ensure(torch.arange(100, dtype=torch.int32, device=gpu)[None], session)
    physical = pool.ensure(torch.arange(64, dtype=torch.int32, device=gpu)[None], session)
    assert sorted(physical[0].tolist()) == list(range(1, 65))


def test_unwritten_and_excess_candidate_ids_map_to_padding(gpu):
    """Ids at or past ``written`` come back as -1 (and flag the status word),
    so attention never reads a stale candidate row; a transient suffix larger
    than the candidate rows is rejected before launch
    (cache/sparse_token_cache.py:254-256)."""
    from cxldsagr_amd.token_pool import TokenPool

    gen = torch.Generator().manual_seed(12)
    pool = TokenPool(1024, 256, device=gpu, candidate_slots=8)
    session = pool.allocate_session(1024)
    pool.write_history(session, torch.randn(500, 576, generator=gen).bfloat16().to(gpu))
    pool.write_candidates(torch.randn(8, 576, generator=gen).bfloat16().to(gpu))
    sel = torch.tensor([[0, 10, 500, 505, 506, 507, 600, -1]], dtype=torch.int32, device=gpu)
    physical = pool.ensure(sel, session, written=506, transient_start=500)
    torch.cuda.synchronize()
    got = physical[0].tolist()
    assert got[2:4] == [pool.slots + 1, pool.slots + 6]
    assert got[4:] == [-1, -1, -1, -1], got
    with pytest.raises(ValueError, match="unwritten"):
        pool.check_status()
    assert pool.check_status() == 0
    with pytest.raises(ValueError, match="candidate slot capacity"):
        pool.ensure(sel, session, written=509, transient_start=500)


def _offload_inputs(gpu, history, queries, seed):
    from cxldsagr_amd.workloads import make_layer_inputs

    inputs = make_layer_inputs(history, queries, seed=seed)
    return inputs, {name: getattr(inputs, name).to(gpu) for name in
                    ("index_q", "index_k", "weights", "mla_q", "kv")}


def test_offload_layer_splits_queries_and_matches_resident_layer(gpu):
    """A9 offload: recall -> sparse_mla_from_pool, the query batch halved while
    the selection's union exceeds the pool (attention.py:213-228). Output bits
    equal the resident fp8 paged layer on the same selection."""
    from cxldsagr_amd.layer import DSALayer, OffloadDSALayer
    from cxldsagr_amd.token_pool import TokenPool

    history, queries = 8192, 16
    inputs, x = _offload_inputs(gpu, history, queries, seed=21)
    tokens = history + queries
    resident = DSALayer(tokens, device=gpu, kv_format="fp8_paged", page_table=inputs.page_table)
    resident.write_history(x["index_k"][:history], x["kv"][:history])
    out_r, sel_r = resident.forward(x["index_q"], x["index_k"][history:], x["weights"],
                                    x["mla_q"], x["kv"][history:])

    pool = TokenPool(tokens + 64 - tokens % 64, 3072, device=gpu, history_capacity=tokens)
    session = pool.allocate_session(tokens)
    layer = OffloadDSALayer(pool, session, tokens)
    layer.write_history(x["index_k"][:history], x["kv"][:history])
    out_o, sel_o = layer.forward(x["index_q"], x["index_k"][history:], x["weights"],
                                 x["mla_q"], x["kv"][history:])
    torch.cuda.synchronize()
    assert torch.equal(sel_o.token_ids, sel_r.token_ids)
    assert bool((sel_o.token_ids >= 0).all())
    assert layer.capacity_splits >= 1
    assert pool.check_status() == 0
    assert torch.equal(out_o.view(torch.int16), out_r.view(torch.int16))


def test_offload_layer_transient_candidates(gpu):
    """GR candidate step: the batch's KV sits in the candidate rows, history is
    not extended, and the output equals the resident layer's."""
    from cxldsagr_amd.layer import DSALayer, OffloadDSALayer
    from cxldsagr_amd.token_pool import TokenPool

    history, queries = 4096, 64
    inputs, x = _offload_inputs(gpu, history, queries, seed=22)
    tokens = history + queries
    resident = DSALayer(tokens, device=gpu, kv_format="fp8_paged", page_table=inputs.page_table)
    resident.write_history(x["index_k"][:history], x["kv"][:history])
    out_r, sel_r = resident.forward(x["index_q"], x["index_k"][history:], x["weights"],
                                    x["mla_q"], x["kv"][history:])
    pool = TokenPool(8192, 8192, device=gpu, candidate_slots=queries)
    session = pool.allocate_session(tokens)
    layer = OffloadDSALayer(pool, session, tokens)
    layer.write_history(x["index_k"][:history], x["kv"][:history])
    out_o, sel_o = layer.forward(x["index_q"], x["index_k"][history:], x["weights"],
                                 x["mla_q"], x["kv"][history:], transient=True)
    torch.cuda.synchronize()
    assert session.written == history
    assert layer.capacity_splits == 0 and pool.check_status() == 0
    assert torch.equal(sel_o.token_ids, sel_r.token_ids)
    ids = sel_o.token_ids
    assert bool((ids >= 0).all()) and bool((ids >= history).any()) and bool((ids < history).any())
    assert torch.equal(out_o.view(torch.int16), out_r.view(torch.int16))


def test_offload_single_query_that_cannot_fit_raises(gpu):
    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.token_pool import TokenPool

    history, queries = 4096, 1
    _, x = _offload_inputs(gpu, history, queries, seed=23)
    pool = TokenPool(4160, 1024, device=gpu)
    session = pool.allocate_session(4160)
    layer = OffloadDSALayer(pool, session, history + queries)
    layer.write_history(x["index_k"][:history], x["kv"][:history])
    with pytest.raises(ValueError, match="at least one query"):
        layer.forward(x["index_q"], x["index_k"][history:], x["weights"], x["mla_q"],
                      x["kv"][history:])
