"""Fused indexer top-k: the logits kernel's radix-digit counts
(``dsa_indexer_logits_fp8_counted``), the top-k that starts from them
(``dsa_topk_radix_digits``) and the two fused (``dsa_indexer_topk_fp8``,
``indexer.logits_topk``), against the unfused entry points and the oracle.

The counts must equal ``oracle.topk.digit_counts`` of the scores exactly; the
top-k results must equal the one-work-group top-k (``dsa_topk_radix``) bit for
bit, and the counts array must be all zero after every top-k call.
"""

import numpy as np
import pytest
import torch

from oracle import topk as otopk

pytestmark = pytest.mark.gpu


def _logit_inputs(rows, columns, device, seed=521):
    torch.manual_seed(seed)
    q = torch.randn(rows, 64, 128).to(torch.float8_e4m3fn).to(device)
    k = torch.randn(columns, 128).to(torch.float8_e4m3fn).to(device)
    weights = (torch.randn(rows, 64) / 64).to(device)
    scales = (torch.rand(columns) + 0.5).to(device)
    return q, k, weights, scales


def _counted_logits(q, k, w, s, query_start, bounds=None, counts=None):
    from cxldsagr_amd import _native
    from cxldsagr_amd.indexer import padded_columns

    rows, columns, device = len(q), len(k), q.device
    out = torch.empty(rows, padded_columns(columns), device=device)
    if counts is None:
        counts = torch.zeros(rows, 2048, dtype=torch.int32, device=device)
    starts, ends = bounds if bounds is not None else (None, None)
    with torch.cuda.device(device):
        _native.call("dsa_indexer_logits_fp8_counted", _native.ptr(q), _native.ptr(k),
                     _native.ptr(w), _native.ptr(s), _native.ptr(starts), _native.ptr(ends),
                     query_start, rows, columns, out.shape[1], None, _native.ptr(out),
                     _native.ptr(counts), _native.stream_of(device))
    return out, counts


def _one_part_topk(scores, columns, k):
    from cxldsagr_amd import _native

    rows, device = len(scores), scores.device
    count = min(k, columns)
    values = torch.empty(rows, count, device=device)
    ids = torch.empty(rows, count, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        _native.call("dsa_topk_radix", _native.ptr(scores), rows, columns, scores.stride(0), k,
                     _native.ptr(values), _native.ptr(ids), count, _native.stream_of(device))
    return values, ids


def _workspace(rows, columns, device):
    """Zeroed workspace of the digit top-k and its [rows, 2048] counts view."""
    import ctypes

    from cxldsagr_amd import _native

    needed = ctypes.c_int64()
    _native.call("dsa_indexer_topk_workspace_bytes", rows, columns, ctypes.byref(needed))
    workspace = torch.zeros(needed.value, dtype=torch.uint8, device=device)
    counts = workspace[:rows * 2048 * 4].view(torch.int32).view(rows, 2048)
    return workspace, counts


def _digits_topk(scores, columns, k, workspace):
    from cxldsagr_amd import _native

    rows, device = len(scores), scores.device
    count = min(k, columns)
    values = torch.empty(rows, count, device=device)
    ids = torch.empty(rows, count, dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        _native.call("dsa_topk_radix_digits", _native.ptr(scores), rows, columns,
                     scores.stride(0), k, _native.ptr(values), _native.ptr(ids), count,
                     _native.ptr(workspace), workspace.numel(), _native.stream_of(device))
    return values, ids


def _ragged_bounds(rows, columns, device, seed):
    g = torch.Generator().manual_seed(seed)
    ends = torch.randint(1, columns + 1, (rows,), generator=g)
    starts = (ends - torch.randint(1, columns + 1, (rows,), generator=g)).clamp_min(0)
    ends[0], starts[0] = columns, 0
    return starts.int().to(device), ends.int().to(device)


@pytest.mark.parametrize(
    "rows,columns,query_start,ragged",
    [(1, 17, 16, False), (5, 4099, 4094, False), (17, 4099, 0, False), (33, 65, 3, False),
     (128, 4224, 4096, False), (40, 3000, 2960, True), (3, 200003, 200000, False),
     (128, 65664, 65536, False)],
)
def test_counted_logits_bits_and_counts(gpu, rows, columns, query_start, ragged):
    from cxldsagr_amd.indexer import logits

    q, k, w, s = _logit_inputs(rows, columns, gpu, seed=rows + columns)
    bounds = _ragged_bounds(rows, columns, gpu, columns) if ragged else None
    plain = logits(q, k, w, s, query_start, _bounds=bounds, _pad_to_stride=True)
    out, counts = _counted_logits(q, k, w, s, query_start, bounds)
    assert counts.data_ptr() % 8 == 0
    assert torch.equal(out.view(torch.int32), plain.view(torch.int32))
    expected = otopk.digit_counts(plain[:, :columns].cpu().numpy())
    np.testing.assert_array_equal(counts.cpu().numpy().astype(np.int64), expected)
    # A second call adds its counts to the first.
    _counted_logits(q, k, w, s, query_start, bounds, counts)
    np.testing.assert_array_equal(counts.cpu().numpy().astype(np.int64), 2 * expected)


def test_counted_logits_nonfinite_scores(gpu):
    """NaN and inf keys give NaN / inf scores; they are counted by their radix
    digit like every other score."""
    from cxldsagr_amd.indexer import logits

    rows, columns = 20, 5000
    q, k, w, s = _logit_inputs(rows, columns, gpu, seed=3)
    codes = k.view(torch.uint8)
    codes[17, 3] = 0x7F  # e4m3fn NaN
    codes[4000, :] = 0x7E  # 448 in every dim: large finite scores
    s[2000] = float("inf")
    plain = logits(q, k, w, s, columns - rows, _pad_to_stride=True)
    out, counts = _counted_logits(q, k, w, s, columns - rows)
    assert torch.equal(out.view(torch.int32), plain.view(torch.int32))
    host = plain[:, :columns].cpu().numpy()
    assert np.isnan(host).any()
    np.testing.assert_array_equal(counts.cpu().numpy().astype(np.int64), otopk.digit_counts(host))


@pytest.mark.parametrize("rows,columns,k", [(1, 1, 1), (3, 17, 2048), (5, 257, 32), (32, 4099, 1024),
                                             (24, 66560, 2048), (4, 69633, 2048), (8, 131584, 2048)])
def test_digits_topk_equals_one_part_kernel(gpu, rows, columns, k):
    generator = torch.Generator(device="cuda").manual_seed(columns + k)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    start = max(0, columns - rows)
    ends = (start + torch.arange(rows, device=gpu) + 1).clamp_max(columns)
    scores.masked_fill_(torch.arange(columns, device=gpu)[None] >= ends[:, None], -torch.inf)
    scores[0, ::3] = 0.25  # ties
    if rows > 2:
        scores[1, 10:20] = -0.0
        scores[2].fill_(-torch.inf)
    values, ids = _one_part_topk(scores, columns, k)
    workspace, counts = _workspace(rows, columns, gpu)
    expected = torch.from_numpy(otopk.digit_counts(scores.cpu().numpy()).astype(np.int32)).to(gpu)
    for with_counts in (True, True, False):  # without counts every row selects from its scores
        if with_counts:
            counts.copy_(expected)
        got_values, got_ids = _digits_topk(scores, columns, k, workspace)
        assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
        assert torch.equal(got_ids, ids)
        assert not counts.any()


def test_digits_topk_past_64_select_parts(gpu):
    """Rows longer than 64 select parts (2,211,840 columns): the parts are not
    listed and the finish selects each row alone from its scores, with the
    threshold digit from the counts."""
    rows, columns, k = 3, 2_300_001, 2048
    generator = torch.Generator(device="cuda").manual_seed(2300)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    scores[0, 1_000_000:1_000_100] = 9.0         # ties at the top, SMALL order
    scores[1, 2_250_000:] = -torch.inf           # a masked tail past part 64
    scores[2] = -scores[2].abs()                 # a negative threshold
    values, ids = _one_part_topk(scores, columns, k)
    workspace, counts = _workspace(rows, columns, gpu)
    host = scores.cpu().numpy()
    expected = torch.from_numpy(otopk.digit_counts(host).astype(np.int32)).to(gpu)
    for _ in range(2):
        counts.copy_(expected)
        got_values, got_ids = _digits_topk(scores, columns, k, workspace)
        assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
        assert torch.equal(got_ids, ids)
        assert not counts.any()
    ref_values, ref_ids = otopk.exact_topk(host, k)
    np.testing.assert_array_equal(got_ids.cpu().numpy(), ref_ids)
    np.testing.assert_array_equal(got_values.cpu().numpy().view(np.uint32), ref_values.view(np.uint32))


def _digit_histogram(scores, columns):
    """[rows, 2048] counts of the radix digits (radix key >> 21) of the first
    ``columns`` scores of each row, on the GPU (torch.bincount)."""
    rows = len(scores)
    bits = scores[:, :columns].contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    keys = torch.where(bits >= 2**31, bits ^ 0xFFFFFFFF, bits | 2**31)
    flat = (keys >> 21) + torch.arange(rows, device=scores.device)[:, None] * 2048
    del bits, keys
    return torch.bincount(flat.view(-1), minlength=rows * 2048).view(rows, 2048)


def test_counted_logits_capped_split(gpu):
    """4,096 rows over 66,000 keys: one key split per query group would span
    66,048 keys, past what the 16-bit LDS counters hold (65,408), so the
    launcher caps the split and the row takes two. Scores equal the plain
    kernel's, counts equal a histogram of them."""
    from cxldsagr_amd.indexer import logits

    rows, columns = 4096, 66_000
    q, k, w, s = _logit_inputs(rows, columns, gpu, seed=4096)
    plain = logits(q, k, w, s, columns - rows, _pad_to_stride=True)
    out, counts = _counted_logits(q, k, w, s, columns - rows)
    assert torch.equal(out.view(torch.int32), plain.view(torch.int32))
    del out
    expected = _digit_histogram(plain, columns)
    assert torch.equal(counts.to(torch.int64), expected)
    assert (counts.sum(dim=1) == columns).all()


def test_digits_topk_ignores_counts_that_do_not_sum_to_the_row(gpu):
    rows, columns, k = 6, 65664, 2048
    generator = torch.Generator(device="cuda").manual_seed(77)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    values, ids = _one_part_topk(scores, columns, k)
    workspace, counts = _workspace(rows, columns, gpu)
    counts.copy_(torch.from_numpy(otopk.digit_counts(scores.cpu().numpy()).astype(np.int32)))
    counts[0, 1000] += 1  # one too many
    counts[1] = 0         # none (a row the logits kernel did not count)
    got_values, got_ids = _digits_topk(scores, columns, k, workspace)
    assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
    assert torch.equal(got_ids, ids)
    assert not counts.any()


def test_digits_topk_bucket_beyond_the_lds_list(gpu):
    """A threshold bucket larger than the LDS refine list (ties over most of a
    row) is split over the row itself."""
    rows, columns, k = 4, 65664, 2048
    generator = torch.Generator(device="cuda").manual_seed(78)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    scores[0, 100:40000] = 1.0   # 39,900 equal keys around the threshold
    scores[1, :] = 0.0
    scores[2, 5:] = -torch.inf
    scores[3, ::2] = 3.0 + torch.arange(0, columns, 2, device=gpu) * 1e-7
    values, ids = _one_part_topk(scores, columns, k)
    workspace, counts = _workspace(rows, columns, gpu)
    counts.copy_(torch.from_numpy(otopk.digit_counts(scores.cpu().numpy()).astype(np.int32)))
    got_values, got_ids = _digits_topk(scores, columns, k, workspace)
    assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
    assert torch.equal(got_ids, ids)
    assert not counts.any()


def test_digits_topk_wave_staging_overflow(gpu):
    """Candidates concentrated in the columns one wave of the select launch
    reads (2,304 of them, past the 1,024 a wave stages) while the row's
    candidates still fit its list: the part is not listed and the finish
    selects the row from its scores. At 65,664 columns the select launch has
    two parts of 32,832 columns; wave 1 of a part reads its columns
    3840 g + [0, 256), g = 0..8."""
    rows, columns, k = 3, 65664, 2048
    generator = torch.Generator(device="cuda").manual_seed(79)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    local = torch.arange(columns, device=gpu) % 32832
    wave1 = (local % 3840) < 256
    assert int(wave1.sum()) == 2 * 2304
    scores[0, wave1] = 5.0 + torch.arange(2 * 2304, device=gpu, dtype=torch.float32) * 1e-6
    scores[1, wave1] = 5.0  # ties: the SMALL order decides
    # A negative threshold (the staging's general radix-key compare).
    scores[2] = -scores[2].abs() - 2.0
    scores[2, wave1] = -0.5 - torch.arange(2 * 2304, device=gpu, dtype=torch.float32) * 1e-6
    values, ids = _one_part_topk(scores, columns, k)
    workspace, counts = _workspace(rows, columns, gpu)
    expected = torch.from_numpy(otopk.digit_counts(scores.cpu().numpy()).astype(np.int32)).to(gpu)
    for _ in range(2):
        counts.copy_(expected)
        got_values, got_ids = _digits_topk(scores, columns, k, workspace)
        assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
        assert torch.equal(got_ids, ids)
        assert not counts.any()
    ref_values, ref_ids = otopk.exact_topk(scores.cpu().numpy(), k)
    np.testing.assert_array_equal(got_ids.cpu().numpy(), ref_ids)
    np.testing.assert_array_equal(got_values.cpu().numpy().view(np.uint32), ref_values.view(np.uint32))


@pytest.mark.parametrize(
    "rows,columns,query_start,topk,ragged",
    [(128, 65664, 65536, 2048, False), (5, 4099, 4094, 2048, False), (3, 1000, 997, 2048, False),
     (40, 3000, 2960, 256, True), (16, 131584, 131568, 2048, False), (1, 1, 0, 1, False)],
)
def test_logits_topk_equals_unfused(gpu, rows, columns, query_start, topk, ragged):
    from cxldsagr_amd import indexer

    q, k, w, s = _logit_inputs(rows, columns, gpu, seed=columns + topk)
    bounds = _ragged_bounds(rows, columns, gpu, rows) if ragged else None
    plain = indexer.logits(q, k, w, s, query_start, _bounds=bounds, _pad_to_stride=True)
    values, ids = _one_part_topk(plain, columns, topk)
    for _ in range(3):
        scores, got_values, got_ids = indexer.logits_topk(q, k, w, s, query_start, topk,
                                                          _bounds=bounds)
        assert torch.equal(scores.view(torch.int32), plain.view(torch.int32))
        assert torch.equal(got_values.view(torch.int32), values.view(torch.int32))
        assert torch.equal(got_ids, ids)
    # The counts of this stream's workspace (its first rows * 8192 bytes) are zero again.
    from cxldsagr_amd import _native

    workspace, layout_rows = indexer._DIGIT_WORKSPACES[(gpu.index, _native.stream_of(gpu).value)]
    assert layout_rows == rows and not workspace[:rows * 2048 * 4].any()
    # Parity with the oracle's top-k of the same scores.
    ref_values, ref_ids = otopk.exact_topk(plain[:, :columns].cpu().numpy(), topk)
    np.testing.assert_array_equal(got_ids.cpu().numpy(), ref_ids)
    np.testing.assert_array_equal(got_values.cpu().numpy().view(np.uint32), ref_values.view(np.uint32))


def test_logits_topk_rejections(gpu):
    from cxldsagr_amd import _native, indexer

    q, k, w, s = _logit_inputs(4, 300, gpu)
    for bad in (0, 2049, True, 1.5):
        with pytest.raises(ValueError, match="k must"):
            indexer.logits_topk(q, k, w, s, 296, bad)
    scores = torch.empty(4, 512, device=gpu)
    values = torch.empty(4, 300, device=gpu)
    ids = torch.empty(4, 300, dtype=torch.int32, device=gpu)
    short = torch.zeros(4 * 2048 * 4 + 4 * 32, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="workspace too small"):
        _native.call("dsa_indexer_topk_fp8", _native.ptr(q), _native.ptr(k), _native.ptr(w),
                     _native.ptr(s), None, None, 296, 4, 300, 512, None, _native.ptr(scores), 2048,
                     _native.ptr(values), _native.ptr(ids), 300, _native.ptr(short), short.numel(),
                     _native.stream_of(gpu))


def test_digits_topk_workspace_reused_across_row_counts(gpu):
    """One workspace for calls whose row counts change (its layout depends on
    them): a call after one with fewer rows finds the earlier call's lists
    where its counts and fill go. Given the zeroing on a layout change (what
    ``logits_topk`` does), every call selects from its counts; without it the
    rows whose counts read stale select from their scores, with the same
    results."""
    columns, k = 65664, 2048
    workspace, _ = _workspace(128, columns, gpu)
    generator = torch.Generator(device="cuda").manual_seed(12)
    for zero in (True, False):
        for rows in (128, 5, 3, 40, 16, 128):
            scores = torch.randn(rows, columns, device=gpu, generator=generator)
            values, ids = _one_part_topk(scores, columns, k)
            if zero:
                workspace.zero_()
            counts = workspace[:rows * 2048 * 4].view(torch.int32).view(rows, 2048)
            counts += torch.from_numpy(otopk.digit_counts(scores.cpu().numpy()).astype(np.int32)).to(gpu)
            got_values, got_ids = _digits_topk(scores, columns, k, workspace)
            assert torch.equal(got_values.view(torch.int32), values.view(torch.int32)), (zero, rows)
            assert torch.equal(got_ids, ids), (zero, rows)
            assert not counts.any()
