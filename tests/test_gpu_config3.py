"""BASELINE config 3 at its real size: 16 users x 65,536 history tokens in a
pinned host arena (1,048,576 fp8 records), one HBM pool of 25 % of all history
(262,144 slots) plus 128 candidate rows, two rounds of 128 fresh transient
candidate tokens per user.

Per user and round: indexer over the user's resident index keys -> top-2048
-> exact recall of the selection into the shared pool -> sparse MLA over the
pool (``OffloadDSALayer.forward(..., transient=True)``). Checked:

* the pool output equals, bit for bit, sparse MLA over a fully resident fp8
  paged cache of the same user's records on the same selection - so every
  selected id resolved to a record byte-equal to its host row;
* after each round the device maps satisfy the reference pool's invariants
  (cache/tests/test_sparse_token_pool.py:32-44, restated as
  ``oracle.recall.check_maps``): sentinel slot, h2d/d2h inverse, free slots
  at priority -1, live priorities below the clock, live records equal to
  their host rows;
* the first user's recall from the cold pool, and the same user's recall in
  round 2 from the full pool (a warm recall that evicts other users'
  records: the oracle's pool is mirrored from the device state just before
  it), leave the same h2d, d2h, priority and record state as the oracle's
  recall of the same selection.
"""

import numpy as np
import pytest
import torch

from oracle import recall as orecall

pytestmark = pytest.mark.gpu

USERS, HISTORY, QUERIES, TOPK = 16, 65536, 128, 2048
SLOTS = USERS * HISTORY // 4


def _host_state(pool):
    return (pool.h2d.cpu().numpy().astype(np.int64), pool.d2h.cpu().numpy(),
            pool.priority.cpu().numpy())


def _check_maps(pool):
    """``oracle.recall.check_maps`` on the device pool, with the record
    comparison done on the device (172 MB of live records)."""
    h2d, d2h, priority = _host_state(pool)
    live = np.nonzero(d2h != orecall.MISSING)[0]
    expected = pool.host[torch.from_numpy(d2h[live])].to(pool.device)
    got = pool.records.view(-1, 656)[torch.from_numpy(live).to(pool.device)]
    assert torch.equal(got, expected)
    assert d2h[0] == orecall.MISSING and priority[0] == orecall.MISSING
    assert np.array_equal(h2d[d2h[live]], live)
    host_live = np.nonzero(h2d != orecall.MISSING)[0]
    assert np.array_equal(d2h[h2d[host_live]], host_live)
    free = d2h[1:] == orecall.MISSING
    assert (priority[1:][free] == -1).all()
    assert (priority[live] < pool.clock).all()
    return len(live)


def test_config3_multi_user_two_rounds(gpu):
    from cxldsagr_amd.attention import pack_kv_fp8, sparse_mla_fp8_paged
    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    tokens = HISTORY + QUERIES
    pool = TokenPool(USERS * HISTORY, SLOTS, device=gpu, candidate_slots=QUERIES,
                     history_capacity=HISTORY)
    pages = (tokens + 63) // 64
    identity = torch.arange(pages, dtype=torch.int32, device=gpu)
    users = []
    for u in range(USERS):
        inputs = make_layer_inputs(HISTORY, QUERIES, seed=947 + u)
        session = pool.allocate_session(HISTORY)
        layer = OffloadDSALayer(pool, session, tokens)
        kv = inputs.kv[:HISTORY].to(gpu)
        layer.write_history(inputs.index_k[:HISTORY].to(gpu), kv)
        resident = torch.zeros(pages, 64, 656, dtype=torch.uint8, device=gpu)
        pack_kv_fp8(kv, resident, identity)
        users.append((layer, resident))
        del inputs, kv
    torch.cuda.synchronize()
    print(f"config3: {USERS} users written, pool {SLOTS} slots", flush=True)

    for rnd in range(2):
        for u, (layer, resident) in enumerate(users):
            fresh = make_layer_inputs(0, QUERIES, seed=100_000 * (rnd + 1) + u)
            x = {name: getattr(fresh, name).to(gpu) for name in
                 ("index_q", "index_k", "weights", "mla_q", "kv")}
            if u == 0:
                mirror = orecall.Pool(pool.host_capacity, SLOTS, 656, QUERIES)
                mirror.host[:] = pool.host.numpy()
                if rnd == 1:
                    # The device pool's state before this warm recall.
                    h2d, d2h, priority = _host_state(pool)
                    mirror.h2d[:], mirror.d2h[:], mirror.priority[:] = h2d, d2h, priority
                    records = pool.records.view(-1, 656)[:len(mirror.records)].cpu().numpy()
                    mirror.records[:] = records
                    mirror.clock = pool.clock
                    free_before = int((d2h[1:] == orecall.MISSING).sum())
                    recalled_before = mirror.recalled
                    del records
            out, selection = layer.forward(x["index_q"], x["index_k"], x["weights"], x["mla_q"],
                                           x["kv"], transient=True)
            pack_kv_fp8(x["kv"], resident, identity, token_offset=HISTORY)
            expected = sparse_mla_fp8_paged(x["mla_q"], resident, identity, selection.token_ids,
                                            576**-0.5, n_tokens=tokens)
            torch.cuda.synchronize()
            assert pool.check_status() == 0
            assert layer.session.written == HISTORY
            # Every row selects TOPK real tokens (no padding, no non-finite score).
            assert bool((selection.token_ids >= 0).all())
            assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), (rnd, u)
            if u == 0:
                ids = selection.token_ids.cpu().numpy()
                table = layer.session.page_table.cpu().numpy()
                orecall.ensure(mirror, ids, table, written=tokens, transient_start=HISTORY)
                if rnd == 1:
                    misses = mirror.recalled - recalled_before
                    print(f"config3 round 2 user 0: {misses} misses, {free_before} free slots",
                          flush=True)
                    assert misses > free_before, "the warm recall must evict"
                h2d, d2h, priority = _host_state(pool)
                np.testing.assert_array_equal(h2d, mirror.h2d)
                np.testing.assert_array_equal(d2h, mirror.d2h)
                np.testing.assert_array_equal(priority, mirror.priority)
                live = np.nonzero(d2h != orecall.MISSING)[0]
                got = pool.records.view(-1, 656)[torch.from_numpy(live).to(gpu)].cpu().numpy()
                np.testing.assert_array_equal(got, mirror.records[live])
                del mirror
        live = _check_maps(pool)
        metrics = pool.metrics()
        print(f"config3 round {rnd + 1}: live slots {live}, recalled so far "
              f"{metrics['recalled_records']}, evicted {metrics['evicted_records']}", flush=True)
        assert 0 < live <= SLOTS
    # 16 users x ~64K selected history each cannot stay resident in 262,144 slots.
    assert pool.metrics()["evicted_records"] > 0
    assert pool.metrics()["recalled_records"] > SLOTS
