"""Multi-user GR serving on the GPU (``cxldsagr_amd.serving.GRServingRunner``):
LRU admission over a host arena that holds two users, transient candidate
steps, a committed append with host write-back, session release.

Every request's output equals, bit for bit, sparse MLA over a fully resident
fp8 paged cache of that user's records on the same selection, so every
selected id resolved to its own record even after the user's host pages were
released and reused by another user. After the sequence the pool maps satisfy
the reference pool's invariants (cache/tests/test_sparse_token_pool.py:32-44),
with every live slot byte-equal to its current host row. The committed
append's host rows equal the oracle's 656-byte records.
"""

import numpy as np
import pytest
import torch

from oracle import kv_fp8 as okv
from oracle import recall as orecall

pytestmark = pytest.mark.gpu

HISTORY, QUERIES, TOPK, LAYERS = 4096, 128, 2048, 2
SLOTS = 4300   # every selection's history union fits: no query split here


def _check_maps(pool):
    h2d = pool.h2d.cpu().numpy().astype(np.int64)
    d2h, priority = pool.d2h.cpu().numpy(), pool.priority.cpu().numpy()
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


class Users:
    """Seeded per-user, per-layer history and candidate batches."""

    def __init__(self, gpu):
        from cxldsagr_amd.workloads import make_layer_inputs

        self.gpu, self.make = gpu, make_layer_inputs

    def history(self, user):
        def build():
            out = []
            for layer in range(LAYERS):
                x = self.make(HISTORY, QUERIES, seed=1000 * user + layer)
                out.append((x.index_k[:HISTORY].to(self.gpu), x.kv[:HISTORY].to(self.gpu)))
            return out
        return build

    def history_kv(self, user, layer):
        return self.make(HISTORY, QUERIES, seed=1000 * user + layer).kv[:HISTORY].to(self.gpu)

    def candidates(self, user, visit):
        out = []
        for layer in range(LAYERS):
            x = self.make(0, QUERIES, seed=77_000 + 100 * user + 10 * visit + layer)
            out.append(tuple(getattr(x, n).to(self.gpu) for n in
                             ("index_q", "index_k", "weights", "mla_q", "kv")))
        return out


def _resident_reference(gpu, kv_tokens, selection, q):
    from cxldsagr_amd.attention import pack_kv_fp8, sparse_mla_fp8_paged

    pages = (len(kv_tokens) + 63) // 64
    identity = torch.arange(pages, dtype=torch.int32, device=gpu)
    cache = torch.zeros(pages, 64, 656, dtype=torch.uint8, device=gpu)
    pack_kv_fp8(kv_tokens, cache, identity)
    return sparse_mla_fp8_paged(q, cache, identity, selection.token_ids, 576 ** -0.5,
                                n_tokens=len(kv_tokens))


def test_lru_admission_transient_steps_and_release(gpu):
    from cxldsagr_amd.serving import GRServingRunner
    from cxldsagr_amd.token_pool import TokenPool

    # Arena: two users of 4096 history tokens (plus a committed batch) fit.
    arena = 2 * HISTORY + 2 * 64 * 2
    pools = [TokenPool(arena, SLOTS, device=gpu, candidate_slots=QUERIES,
                       history_capacity=HISTORY + QUERIES) for _ in range(LAYERS)]
    users = Users(gpu)
    plan = [(0, False), (1, False), (0, True), (2, False), (1, False), (2, True), (0, False)]
    expected_evicted = {3: (1,), 4: (0,), 6: (1,)}
    visits = {}
    with GRServingRunner(pools, topk=TOPK) as runner:
        for step, (user, hit) in enumerate(plan):
            visit = visits.get(user, 0)
            visits[user] = visit + 1
            batch = users.candidates(user, visit)
            print(f"serving step {step}: user {user}", flush=True)
            result = runner.execute({"user_id": user, "signature": ("history", user),
                                     "history_tokens": HISTORY, "history": users.history(user),
                                     "candidates": batch})
            m = result.metrics
            assert m["prefix_cache_hit"] == hit, (step, m)
            assert tuple(m["evicted_users"]) == expected_evicted.get(step, ()), (step, m)
            assert m["fetch_bytes"] == 656 * m["recalled_records"]
            if not hit:   # a fresh session's rows are all on the host
                assert m["recalled_records"] > 0
            for layer in range(LAYERS):
                kv = torch.cat((users.history_kv(user, layer), batch[layer][4]))
                ref = _resident_reference(gpu, kv, result.selections[layer], batch[layer][3])
                torch.cuda.synchronize()
                assert bool((result.selections[layer].token_ids >= 0).all())
                assert torch.equal(result.outputs[layer].view(torch.int16), ref.view(torch.int16)), (
                    step, layer)
            assert runner.lru.keys()[-1] == user and len(runner.lru) <= 2
        for pool in pools:
            assert _check_maps(pool) > 0
    # close() released every session: no host row stays mapped.
    for pool in pools:
        assert int((pool.h2d != orecall.MISSING).sum()) == 0
        assert pool.free_host_pages == arena // 64


def test_committed_append_writes_back_and_is_recalled(gpu):
    from cxldsagr_amd.serving import GRServingRunner
    from cxldsagr_amd.token_pool import TokenPool

    pools = [TokenPool(2 * HISTORY, SLOTS, device=gpu, candidate_slots=QUERIES,
                       history_capacity=HISTORY + QUERIES) for _ in range(LAYERS)]
    users = Users(gpu)
    with GRServingRunner(pools, topk=TOPK) as runner:
        first = users.candidates(5, 0)
        result = runner.execute({"user_id": 5, "signature": "h5", "history_tokens": HISTORY,
                                 "history": users.history(5), "candidates": first,
                                 "commit": True, "commit_signature": "h5+1"})
        assert result.metrics["committed"] and not result.metrics["prefix_cache_hit"]
        layers = runner.lru._entries[5].session
        torch.cuda.synchronize()
        for layer, pool in zip(layers, pools):
            assert layer.written == HISTORY + QUERIES
            rows = layer.session.global_rows(HISTORY, HISTORY + QUERIES)
            got = pool.host[rows].numpy()
            kv_bits = first[layer.layer_idx][4].cpu().view(torch.int16).numpy().view(np.uint16)
            np.testing.assert_array_equal(got, okv.encode_records(kv_bits))
        # The extended history hits under its new signature; the committed
        # tokens are recalled like any other history.
        second = users.candidates(5, 1)
        result = runner.execute({"user_id": 5, "signature": "h5+1",
                                 "history_tokens": HISTORY + QUERIES, "history": None,
                                 "candidates": second})
        assert result.metrics["prefix_cache_hit"]
        for layer in range(LAYERS):
            kv = torch.cat((users.history_kv(5, layer), first[layer][4], second[layer][4]))
            ref = _resident_reference(gpu, kv, result.selections[layer], second[layer][3])
            torch.cuda.synchronize()
            ids = result.selections[layer].token_ids
            assert bool(((ids >= HISTORY) & (ids < HISTORY + QUERIES)).any())
            assert torch.equal(result.outputs[layer].view(torch.int16), ref.view(torch.int16))


def test_release_session_frees_slots_and_pages(gpu):
    """TokenPool.release_session against the oracle's release_ids on the same
    pool state."""
    from cxldsagr_amd.token_pool import TokenPool

    pool = TokenPool(4 * 64, 100, device=gpu, candidate_slots=0)
    gen = torch.Generator().manual_seed(3)
    sessions = [pool.allocate_session(128) for _ in range(2)]
    for s in sessions:
        pool.write_history(s, torch.randn(128, 576, generator=gen).bfloat16().to(gpu))
    for s in sessions:
        sel = torch.randint(0, 128, (2, 40), generator=gen).int().to(gpu)
        pool.ensure(sel, s)
    torch.cuda.synchronize()
    mirror = orecall.Pool(pool.host_capacity, pool.slots, 656)
    mirror.h2d = pool.h2d.cpu().numpy().astype(np.int64)
    mirror.d2h, mirror.priority = pool.d2h.cpu().numpy(), pool.priority.cpu().numpy()
    orecall.release_ids(mirror, sessions[0].global_rows(0, 128).numpy())
    free_before = pool.free_host_pages
    pool.release_session(sessions[0])
    np.testing.assert_array_equal(pool.h2d.cpu().numpy().astype(np.int64), mirror.h2d)
    np.testing.assert_array_equal(pool.d2h.cpu().numpy(), mirror.d2h)
    np.testing.assert_array_equal(pool.priority.cpu().numpy(), mirror.priority)
    assert pool.free_host_pages == free_before + 2 and pool.status.item() == 0
    with pytest.raises(ValueError, match="released"):
        pool.ensure(torch.zeros(1, 1, dtype=torch.int32, device=gpu), sessions[0])
    # The freed pages serve a new session whose rows start unmapped.
    fresh = pool.allocate_session(128)
    assert set(fresh.host_pages) == set(sessions[0].host_pages)
    pool.write_history(fresh, torch.randn(128, 576, generator=gen).bfloat16().to(gpu))
    physical = pool.ensure(torch.arange(64, dtype=torch.int32, device=gpu)[None], fresh)
    torch.cuda.synchronize()
    got = pool.records.view(-1, 656)[physical[0].long()]
    assert torch.equal(got.cpu(), pool.host[fresh.global_rows(0, 64)])


def test_failed_requests_discard_the_session_and_budget_errors_evict_nothing(gpu):
    """A request that fails after admission releases its session (the
    reference runner's discard, serving/persistent.py:218-226); a request
    larger than the arena raises before evicting anyone."""
    from cxldsagr_amd.serving import CacheBudgetExceeded, GRServingRunner
    from cxldsagr_amd.token_pool import TokenPool

    pools = [TokenPool(2 * HISTORY, SLOTS, device=gpu, candidate_slots=QUERIES,
                       history_capacity=HISTORY + QUERIES) for _ in range(LAYERS)]
    users = Users(gpu)
    with GRServingRunner(pools, topk=TOPK) as runner:
        runner.execute({"user_id": 0, "signature": "h0", "history_tokens": HISTORY,
                        "history": users.history(0), "candidates": users.candidates(0, 0)})
        free = [pool.free_host_pages for pool in pools]
        # History of the wrong length: fails after admission, session discarded.
        with pytest.raises(ValueError, match="history length"):
            runner.execute({"user_id": 1, "signature": "h1", "history_tokens": HISTORY - 64,
                            "history": users.history(1), "candidates": users.candidates(1, 0)})
        assert runner.lru.keys() == [0]
        assert [pool.free_host_pages for pool in pools] == free
        # More than the whole arena: refused, user 0 stays cached.
        with pytest.raises(CacheBudgetExceeded):
            runner.execute({"user_id": 2, "signature": "h2", "history_tokens": 2 * HISTORY + 64,
                            "history": users.history(2), "candidates": users.candidates(2, 0)})
        assert runner.lru.keys() == [0]
        result = runner.execute({"user_id": 0, "signature": "h0", "history_tokens": HISTORY,
                                 "history": None, "candidates": users.candidates(0, 1)})
        assert result.metrics["prefix_cache_hit"]
        for pool in pools:
            assert pool.check_status() == 0


def test_chunked_requests_equal_resident_attention(gpu):
    """``GRServingRunner(chunks=2)``: each layer's candidate batch runs as two
    chunks of rows whose recalls overlap (``multi_user.ChunkedForward``); on
    pools that hold two histories the pipeline is taken, and every output
    still equals, bit for bit, sparse MLA over a fully resident cache of the
    user's records on the same selection, through a miss, a committed append
    and a hit on the extended history."""
    from cxldsagr_amd.serving import GRServingRunner
    from cxldsagr_amd.token_pool import TokenPool

    grown = HISTORY + QUERIES
    pools = [TokenPool(2 * grown, 2 * grown, device=gpu, candidate_slots=QUERIES,
                       history_capacity=grown) for _ in range(LAYERS)]
    users = Users(gpu)
    with GRServingRunner(pools, topk=TOPK, chunks=2) as runner:
        first = users.candidates(4, 0)
        print("chunked serving: miss with commit", flush=True)
        result = runner.execute({"user_id": 4, "signature": "h4", "history_tokens": HISTORY,
                                 "history": users.history(4), "candidates": first,
                                 "commit": True, "commit_signature": "h4+1"})
        layers = runner.lru._entries[4].session
        assert all(runner.pipelines[i].overlaps(layer, QUERIES, transient=True)
                   for i, layer in enumerate(layers))
        for layer in range(LAYERS):
            kv = torch.cat((users.history_kv(4, layer), first[layer][4]))
            ref = _resident_reference(gpu, kv, result.selections[layer], first[layer][3])
            torch.cuda.synchronize()
            assert torch.equal(result.outputs[layer].view(torch.int16), ref.view(torch.int16))
        second = users.candidates(4, 1)
        print("chunked serving: hit, transient", flush=True)
        result = runner.execute({"user_id": 4, "signature": "h4+1", "history_tokens": grown,
                                 "history": None, "candidates": second})
        assert result.metrics["prefix_cache_hit"]
        for layer in range(LAYERS):
            kv = torch.cat((users.history_kv(4, layer), first[layer][4], second[layer][4]))
            ref = _resident_reference(gpu, kv, result.selections[layer], second[layer][3])
            torch.cuda.synchronize()
            assert torch.equal(result.outputs[layer].view(torch.int16), ref.view(torch.int16))
        for pool in pools:
            assert pool.check_status() == 0
            assert _check_maps(pool) > 0
    with pytest.raises(ValueError, match="chunks"):
        GRServingRunner(pools, chunks=0)
