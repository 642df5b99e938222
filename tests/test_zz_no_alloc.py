"""The allocation-free top-k entry point (dsa_topk_radix_split_static).

Called through the C ABI and compared bit for bit with the workspace entry
point dsa_topk_radix_split on the same scores, on two calls in a row, the
second with fewer rows and columns than the first (the library-owned array
keeps the first call's lists; the second must not read them). Also: the
row limit is rejected with a clear error before any launch, and short rows
(one work-group per row, no scratch) take the same path as the workspace
entry.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu


def _topk(name, scores, k, with_workspace):
    from cxldsagr_amd import _native

    rows, columns = scores.shape
    count = min(k, columns)
    values = torch.empty((rows, count), dtype=torch.float32, device=scores.device)
    ids = torch.empty((rows, count), dtype=torch.int32, device=scores.device)
    stream = _native.stream_of(scores.device)
    args = [_native.ptr(scores), rows, columns, scores.stride(0), k, _native.ptr(values),
            _native.ptr(ids), count]
    if with_workspace:
        size = ctypes.c_int64()
        _native.call("dsa_topk_workspace_bytes", rows, ctypes.byref(size))
        workspace = torch.empty(size.value, dtype=torch.uint8, device=scores.device)
        args += [_native.ptr(workspace), workspace.numel()]
    with torch.cuda.device(scores.device):
        _native.call(name, *args, stream)
    torch.cuda.synchronize()
    return values, ids


def _scores(rows, columns, seed, device):
    gen = torch.Generator().manual_seed(seed)
    scores = torch.randn(rows, columns, generator=gen)
    # ties and masked tails, as the indexer produces them
    scores[:, ::7] = 0.5
    scores[0, columns // 2:] = -float("inf")
    return scores.to(device)


def test_static_topk_equals_workspace_topk_on_two_calls(gpu):
    for rows, columns, seed in ((512, 65792, 1), (128, 20000, 2), (3, 9000, 3), (40, 5000, 4)):
        scores = _scores(rows, columns, seed, gpu)
        v_ref, i_ref = _topk("dsa_topk_radix_split", scores, 2048, True)
        v, i = _topk("dsa_topk_radix_split_static", scores, 2048, False)
        assert torch.equal(v.view(torch.int32), v_ref.view(torch.int32)), (rows, columns)
        assert torch.equal(i, i_ref), (rows, columns)


def test_static_topk_rejects_rows_beyond_the_array(gpu):
    from cxldsagr_amd import _native

    scores = torch.zeros((513, 8192), dtype=torch.float32, device=gpu)
    with pytest.raises(ValueError, match="at most 512 rows"):
        _topk("dsa_topk_radix_split_static", scores, 2048, False)
    assert "512" in _native.last_error()
