"""Zero-row calls through the C ABI.

Each hot-path entry point, given otherwise valid buffers and zero rows (or
zero records), returns status 0 without launching anything and leaves its
outputs untouched; the reference's operators accept empty batches the same
way (``selection.py`` exact top-k of zero rows, ``kv_transfer.py`` gathers
of zero records, ``device_only/mla.py`` of zero queries). A guard value in
every output buffer shows that nothing was written.
"""

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

GUARD = 0x5A


def _lib_call(name, *args):
    from cxldsagr_amd import _native

    _native.call(name, *args)  # raises on a nonzero status


def _guarded(*shape, dtype, gpu):
    t = torch.empty(shape, dtype=torch.uint8, device=gpu).fill_(GUARD)
    return t.view(dtype) if dtype is not torch.uint8 else t


def _untouched(*tensors):
    torch.cuda.synchronize()
    for t in tensors:
        assert bool((t.view(torch.uint8) == GUARD).all())


def test_zero_row_calls_return_ok_and_write_nothing(gpu):
    from cxldsagr_amd import _native as n

    stream = n.stream_of(gpu)
    p = n.ptr
    columns, width = 256, 256
    q8 = torch.zeros((4, 64, 128), dtype=torch.uint8, device=gpu)
    k8 = torch.zeros((columns, 128), dtype=torch.uint8, device=gpu)
    w = torch.zeros((4, 64), dtype=torch.float32, device=gpu)
    ks = torch.ones(columns, dtype=torch.float32, device=gpu)

    # A1: quantise zero rows.
    x = torch.zeros((4, 128), dtype=torch.bfloat16, device=gpu)
    codes = _guarded(4, 128, dtype=torch.uint8, gpu=gpu)
    scales = _guarded(4, dtype=torch.float32, gpu=gpu)
    _lib_call("dsa_quantize_fp8_rows", p(x), 0, 0, 128, 128, p(codes), p(scales), 1, stream)
    _untouched(codes, scales)

    # A4: logits of zero query rows.
    out = _guarded(4, width, dtype=torch.float32, gpu=gpu)
    _lib_call("dsa_indexer_logits_fp8", p(q8), p(k8), p(w), p(ks), None, None, 0, 0, columns,
              width, p(out), stream)
    _untouched(out)

    # A6: top-k of zero rows.
    scores = torch.zeros((4, columns), dtype=torch.float32, device=gpu)
    values = _guarded(4, 64, dtype=torch.float32, gpu=gpu)
    ids = _guarded(4, 64, dtype=torch.int32, gpu=gpu)
    _lib_call("dsa_topk_radix", p(scores), 0, columns, columns, 64, p(values), p(ids), 64, stream)
    _untouched(values, ids)

    # (f)1: the fused indexer step for zero rows.
    size = ctypes.c_int64()
    _lib_call("dsa_indexer_select_workspace_bytes", 4, columns, 0, ctypes.byref(size))
    workspace = torch.zeros(max(size.value, 256), dtype=torch.uint8, device=gpu)
    sel_scores = _guarded(4, width, dtype=torch.float32, gpu=gpu)
    _lib_call("dsa_indexer_select_fp8", p(q8), p(k8), p(w), p(ks), None, None, 0, 0, columns,
              None, p(sel_scores), 64, p(values), p(ids), 64, p(workspace), workspace.numel(),
              stream)
    _untouched(sel_scores, values, ids)

    # A7/A8: sparse MLA over the fp8 paged cache for zero query rows.
    mla_q = torch.zeros((4, 128, 576), dtype=torch.bfloat16, device=gpu)
    cache = torch.zeros((1, 64, 656), dtype=torch.uint8, device=gpu)
    table = torch.zeros(1, dtype=torch.int32, device=gpu)
    sel = torch.zeros((4, 64), dtype=torch.int32, device=gpu)
    mla_out = _guarded(4, 128, 512, dtype=torch.bfloat16, gpu=gpu)
    _lib_call("dsa_sparse_mla_fp8_paged", p(mla_q), 0, 128, p(cache), 1, p(table), 64, p(sel), 64,
              ctypes.c_float(576**-0.5), p(mla_out), stream)
    _untouched(mla_out)

    # A11: a gather of zero records.
    host = torch.zeros((8, 656), dtype=torch.uint8).pin_memory()
    dev = _guarded(8, 656, dtype=torch.uint8, gpu=gpu)
    host_ids = torch.zeros(1, dtype=torch.int64, device=gpu)
    dev_ids = torch.zeros(1, dtype=torch.int64, device=gpu)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    _lib_call("dsa_gather_records", p(host), 8, p(dev), 8, 656, p(host_ids), p(dev_ids), 0, None,
              0, 0, p(status), stream)
    _untouched(dev)
    assert int(status.item()) == 0
