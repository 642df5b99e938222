"""Fused indexer top-k without the score matrix (``indexer.select_topk``,
``dsa_indexer_select_fp8``): per-row floors, the logits kernel writing only
candidates at or above them, the exact top-k of the candidates with a full
recompute of any row the candidates cannot decide.

Every case must equal ``exact_topk(logits(...))`` - the unfused HIP path,
itself pinned to ``oracle.topk`` / ``oracle.logits`` - bit for bit (values
and indices), and the config-1 case also ``oracle.topk.exact_topk`` of the
same scores. The test hooks force each path: floors above the row's
count-th score (recompute), short candidate lists (spills), equal scores
(too many candidates), short rows (no floor).
"""

import numpy as np
import pytest
import torch

from oracle import topk as otopk

pytestmark = pytest.mark.gpu

INF_KEY = np.int32(np.uint32(0xFF800000).view(np.int32))  # radix key of +inf


def _inputs(rows, columns, device, seed=731, heavy=0.05):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(rows, 64, 128, generator=g)
    k = torch.randn(columns, 128, generator=g)
    hot = torch.randperm(columns, generator=g)[: int(heavy * columns)]
    direction = q.mean(dim=(0, 1))
    k[hot] += 2 * direction / direction.norm()
    weights = torch.randn(rows, 64, generator=g) / 8
    scales = torch.rand(columns, generator=g) + 0.5
    return (q.to(torch.float8_e4m3fn).to(device), k.to(torch.float8_e4m3fn).to(device),
            weights.to(device), scales.to(device))


def _unfused(q, k, w, s, query_start, topk, bounds=None):
    from cxldsagr_amd import indexer

    scores = indexer.logits(q, k, w, s, query_start, _bounds=bounds)
    values, ids = indexer.exact_topk(scores, topk)
    return scores, values, ids


def _same(got, want):
    gv, gi = got
    wv, wi = want
    assert gv.shape == wv.shape and gi.shape == wi.shape
    assert torch.equal(gv.view(torch.int32), wv.view(torch.int32)), "values differ"
    assert torch.equal(gi, wi), "indices differ"


def _split_plan(rows, columns, device):
    """The logits launcher's key splits (logits.hip split_plan): (splits, per)."""
    ldo = (columns + 255) // 256 * 256
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    qgroups = (rows + 15) // 16
    splits = max(1, (cus + qgroups - 1) // qgroups)
    per = (ldo + splits - 1) // splits
    per = (per + 127) // 128 * 128
    splits = (ldo + per - 1) // per
    if splits >= 8:
        splits = (splits + 7) // 8 * 8
    return splits, per


def _radix(values):
    bits = values.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    return torch.where(bits >= 2**31, bits ^ 0xFFFFFFFF, bits | 2**31)


@pytest.mark.parametrize(
    "rows,columns,query_start,topk",
    [
        (128, 65664, 65536, 2048),   # config 1
        (40, 30000, 29960, 2048),
        (17, 9000, 8983, 2048),      # visible counts across the no-floor bound (8192)
        (3, 140000, 139997, 1000),
        (24, 50000, 49976, 1),
        # Many rows: one or two key splits per row, so each split's list is
        # served by 1024 or 512 threads of the top-k work-group.
        (2048, 20000, 17952, 2048),
        (4096, 12000, 7904, 2048),
    ],
)
def test_select_equals_unfused(gpu, rows, columns, query_start, topk):
    from cxldsagr_amd import indexer

    q, k, w, s = _inputs(rows, columns, gpu)
    scores, values, ids = _unfused(q, k, w, s, query_start, topk)
    got = indexer.select_topk(q, k, w, s, query_start, topk)
    torch.cuda.synchronize()
    _same(got, (values, ids))
    if rows == 128:
        ref_v, ref_i = otopk.exact_topk(scores.cpu().numpy(), topk)
        assert np.array_equal(got[0].cpu().numpy().view(np.int32), ref_v.view(np.int32))
        assert np.array_equal(got[1].cpu().numpy(), ref_i)


def test_select_config1_lists_only_candidates(gpu):
    """At config 1 every row gets a floor, no split spills, each split lists
    exactly its scores at or above the floor, and a row's candidates (a few
    thousand) contain its top 2048: the score matrix is never written."""
    from cxldsagr_amd import _native, indexer

    rows, columns, query_start, topk = 128, 65664, 65536, 2048
    q, k, w, s = _inputs(rows, columns, gpu, seed=947)
    scores, values, ids = _unfused(q, k, w, s, query_start, topk)
    got = indexer.select_topk(q, k, w, s, query_start, topk)
    torch.cuda.synchronize()
    _same(got, (values, ids))
    workspace, _ = indexer._SELECT_BUFFERS[(gpu.index, _native.stream_of(gpu).value)]
    pair = workspace[:8 * rows].view(torch.int32).view(rows, 2).to(torch.int64) & 0xFFFFFFFF
    floors = pair.min(dim=1).values
    assert (floors != 0).all()
    radix = _radix(scores)
    candidates = radix >= floors[:, None]
    per_row = candidates.sum(dim=1)
    assert (per_row >= topk).all(), "a floor above the row's 2048th score"
    assert per_row.max().item() <= 8192
    assert per_row.sum().item() * 8 <= 6 * 2**20, "more than 6 MiB of candidate keys"
    splits, per = _split_plan(rows, columns, gpu)
    records_at = (8 * rows + 255) // 256 * 256
    rec = workspace[records_at:records_at + rows * splits * 8].view(torch.int32).view(rows, splits, 2)
    live = [sp for sp in range(splits) if sp * per < columns]
    assert (rec[:, live, 1] == 0x7FFFFFFF).all(), "a split spilled"
    for sp in live:
        listed = candidates[:, sp * per:min(columns, (sp + 1) * per)].sum(dim=1)
        assert torch.equal(rec[:, sp, 0].to(torch.int64), listed)


def test_select_forced_recompute(gpu):
    """Floors above the count-th score leave too few candidates: those rows
    are recomputed in the top-k kernel and must match bit for bit."""
    from cxldsagr_amd import indexer

    rows, columns, query_start, topk = 48, 40000, 39952, 2048
    q, k, w, s = _inputs(rows, columns, gpu, seed=17)
    _, values, ids = _unfused(q, k, w, s, query_start, topk)
    floors = indexer.select_floors(q, k, w, s, query_start, topk)
    # Rows 0-15: +inf floor (no candidates); rows 16-31: one above the row's
    # count-th radix key (count - 1 candidates); the rest: estimated floors.
    kth = values[:, -1].contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    kth_radix = torch.where(kth >= 2**31, kth ^ 0xFFFFFFFF, kth | 2**31)
    high = floors.clone()
    high[:16] = int(INF_KEY)
    just_above = (kth_radix[16:32] + 1).to(torch.int64)
    high[16:32] = torch.where(just_above >= 2**31, just_above - 2**32, just_above).to(torch.int32)
    got = indexer.select_topk(q, k, w, s, query_start, topk, _floors=high)
    torch.cuda.synchronize()
    _same(got, (values, ids))


@pytest.mark.parametrize("cap", [0, 512])
def test_select_more_candidates_than_the_sort_holds(gpu, cap):
    """Floors far below the count-th score (~16K candidates per row, more than
    the 8,192 the sort holds): the top-k raises the floor to the threshold
    digit of the candidates and lists again, with the lists spilling (default
    capacity) or holding every candidate (512 slots per split); the result
    must not change."""
    from cxldsagr_amd import indexer

    rows, columns, query_start, topk = 32, 50000, 49968, 2048
    q, k, w, s = _inputs(rows, columns, gpu, seed=16000 + cap)
    scores, values, ids = _unfused(q, k, w, s, query_start, topk)
    low = torch.topk(scores[:, :columns], 16000, dim=1).values[:, -1]
    radix = _radix(low)
    floors = torch.where(radix >= 2**31, radix - 2**32, radix).to(torch.int32)
    got = indexer.select_topk(q, k, w, s, query_start, topk, _floors=floors, _list_cap=cap)
    torch.cuda.synchronize()
    _same(got, (values, ids))


@pytest.mark.parametrize("cap", [64, 128, 192])
def test_select_spills(gpu, cap):
    """Short candidate lists make the splits spill their scores to the score
    scratch part way; the top-k reads the spilled columns back."""
    from cxldsagr_amd import indexer

    rows, columns, query_start, topk = 32, 50000, 49968, 2048
    q, k, w, s = _inputs(rows, columns, gpu, seed=cap)
    _, values, ids = _unfused(q, k, w, s, query_start, topk)
    got = indexer.select_topk(q, k, w, s, query_start, topk, _list_cap=cap)
    torch.cuda.synchronize()
    _same(got, (values, ids))


def test_select_equal_scores_and_bounds(gpu):
    """Zero weights (every score +0.0: every column a candidate, far more than
    the kernel holds), and ragged [starts, ends) bounds including short rows."""
    from cxldsagr_amd import indexer

    rows, columns, query_start, topk = 20, 30000, 29980, 2048
    q, k, w, s = _inputs(rows, columns, gpu, seed=5)
    w[:6] = 0.0
    g = torch.Generator().manual_seed(3)
    ends = torch.randint(1000, columns + 1, (rows,), generator=g)
    starts = (ends - torch.randint(100, columns, (rows,), generator=g)).clamp_min(0)
    ends[0], starts[0] = columns, 0
    bounds = (starts.int().to(gpu), ends.int().to(gpu))
    _, values, ids = _unfused(q, k, w, s, query_start, topk, bounds)
    got = indexer.select_topk(q, k, w, s, query_start, topk, _bounds=bounds)
    torch.cuda.synchronize()
    _same(got, (values, ids))


def test_select_config4_size(gpu):
    """BASELINE config 4's indexer (512 queries over 131,584 keys, heavy
    hitters in 8 contiguous spans): the candidate path against the unfused
    one."""
    from cxldsagr_amd import indexer
    from cxldsagr_amd.workloads import make_layer_inputs

    inputs = make_layer_inputs(131072, 512, heavy_fraction=0.10, spans=8, seed=947)
    q8, qs = indexer.quantize_index(inputs.index_q.to(gpu))
    k8, ks = indexer.quantize_index(inputs.index_k.to(gpu))
    w = (inputs.weights.to(gpu) * qs[..., 0]).contiguous()
    ks = ks[:, 0].contiguous()
    _, values, ids = _unfused(q8, k8, w, ks, 131072, 2048)
    got = indexer.select_topk(q8, k8, w, ks, 131072, 2048)
    torch.cuda.synchronize()
    _same(got, (values, ids))


def test_layer_prologue_floors(gpu):
    """The layer prologue's floors (estimated from the history keys in the
    same launch as the quantisers): every row's 2048th score at or above its
    floor, a few thousand candidates per row, and the layer step's selection
    equal to the unfused top-k of the same scores."""
    from cxldsagr_amd import indexer
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.workloads import make_layer_inputs

    history, queries = 65536, 128
    inputs = make_layer_inputs(history, queries, seed=947)
    layer = DSALayer(history + queries, device=gpu, page_table=inputs.page_table)
    layer.write_history(inputs.index_k[:history].to(gpu), inputs.kv[:history].to(gpu))
    index_q, weights = inputs.index_q.to(gpu), inputs.weights.to(gpu)
    index_k = inputs.index_k[history:].to(gpu).contiguous()
    mla_q, kv = inputs.mla_q.to(gpu), inputs.kv[history:].to(gpu).contiguous()
    floors = torch.zeros((queries, 2), dtype=torch.int32, device=gpu)
    q8, folded, _ = layer._prologue(index_q, index_k, weights, kv, history, floors)
    scores = indexer.logits(q8, layer.index_keys, folded, layer.index_scales, history)
    values, ids = indexer.exact_topk(scores, 2048)
    torch.cuda.synchronize()
    fl = (floors.to(torch.int64) & 0xFFFFFFFF).min(dim=1).values
    assert (fl > 0).all()
    assert (fl <= _radix(values[:, -1])).all(), "a floor above the row's 2048th score"
    per_row = (_radix(scores) >= fl[:, None]).sum(dim=1)
    assert per_row.max().item() <= 8192
    layer.written = history
    _, selection = layer.forward(index_q, index_k, weights, mla_q, kv)
    torch.cuda.synchronize()
    assert torch.equal(selection.token_ids, ids)


@pytest.mark.parametrize("case", range(24))
def test_select_random_shapes_bounds_caps_and_floors(gpu, case):
    """Seeded random cases over every path of the candidate top-k at once:
    row counts 1-300, rows of 1-70K columns, top-k 1-2048, causal or ragged
    bounds, default or short candidate lists (spills), and floors estimated,
    absent, or forced at a random rank of each row's scores (recompute when
    above its count-th score, the raised floor when far below). Every case
    equals the unfused logits -> exact_topk bit for bit."""
    from cxldsagr_amd import indexer

    rng = np.random.default_rng(9000 + case)
    rows = int(rng.integers(1, 301))
    columns = int(rng.integers(max(rows, 16), 70001))
    topk = int(rng.choice([1, 7, 100, 1000, 2048]))
    query_start = columns - rows
    q, k, w, s = _inputs(rows, columns, gpu, seed=100 + case, heavy=float(rng.choice([0.0, 0.05, 0.3])))
    bounds = None
    if rng.random() < 0.4:
        ends = rng.integers(1, columns + 1, rows)
        starts = (ends * rng.random(rows) * 0.5).astype(np.int64)
        bounds = (torch.from_numpy(starts.astype(np.int32)).to(gpu),
                  torch.from_numpy(ends.astype(np.int32)).to(gpu))
    scores, values, ids = _unfused(q, k, w, s, query_start, topk, bounds)
    hooks = {}
    if rng.random() < 0.3:
        hooks["_list_cap"] = int(rng.choice([64, 128, 256, 512]))
    mode = rng.choice(["estimated", "none", "forced"])
    if mode != "estimated":
        keys = _radix(scores[:, :columns])  # -inf columns have the lowest keys
        if mode == "none":
            floors = torch.zeros(rows, dtype=torch.int64, device=gpu)
        else:
            ranks = torch.from_numpy(rng.integers(1, min(columns, 20000) + 1, rows)).to(gpu)
            floors = torch.sort(keys, dim=1, descending=True).values.gather(1, (ranks - 1)[:, None])[:, 0]
        hooks["_floors"] = torch.where(floors >= 2**31, floors - 2**32, floors).to(torch.int32)
    print(f"random select case {case}: rows {rows} columns {columns} topk {topk} bounds "
          f"{bounds is not None} mode {mode} hooks {sorted(hooks)}", flush=True)
    got = indexer.select_topk(q, k, w, s, query_start, topk, _bounds=bounds, **hooks)
    _same(got, (values, ids))
