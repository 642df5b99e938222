"""DSA indexer operators on MI355X: fp8 quantisation, fp8 MQA logits, exact top-k.

Drop-in for the reference's indexer operators (same names, argument order,
validation messages and output layouts):

* ``quantize_index``  - ``operators/deepseek_v32/indexer/quantization.py:63-88``
* ``logits``          - ``operators/deepseek_v32/indexer/echo.py:299-410``
  (resident branch; the fused ECHO prefetch branch ``:412-483`` is replaced by
  the top-k-driven gather in ``cxldsagr_amd.token_pool``)
* ``exact_topk``      - ``operators/deepseek_v32/indexer/selection.py:62-113``
* ``logits_topk``     - ``logits`` then ``exact_topk`` as the indexer step of
  ``models/deepseek_v32/attention.py:338-363`` calls them, fused through the
  logits kernel's radix-digit counts

All work runs in hand-written gfx950 kernels (``csrc/quantize.hip``,
``csrc/logits.hip``, ``csrc/topk.hip``) on the caller's current stream, with
no host synchronisation.
"""

import ctypes

import torch

from cxldsagr_amd import _native

SCORE_ALIGNMENT = 256


def _check_tensor(tensor, shape, dtype, device, name):
    """Mirror of ``echo.py:86-95``."""
    if (
        not isinstance(tensor, torch.Tensor)
        or tuple(tensor.shape) != tuple(shape)
        or tensor.dtype != dtype
        or tensor.device != device
        or not tensor.is_contiguous()
        or tensor.requires_grad
    ):
        raise ValueError(f"{name} must be contiguous {dtype} {tuple(shape)} on {device}")


def quantize_index(x, scale_fmt="ue8m0"):
    """Quantize each last-dimension row, returning contiguous FP8 and FP32 ``[..., 1]``.

    Same arithmetic as the reference device kernel (``quantization.py:34-60``):
    NaN-propagating amax, ``clamp_min(1e-4)``, ``scale = amax * fl32(1/448)``,
    UE8M0 rounds the scale up to a power of two, RNE e4m3fn cast of
    ``clamp(x / scale, -448, 448)``. Accepts bf16, fp16 and fp32 in any layout
    (non-unit last-dim strides are copied first).
    """
    data, scales, _ = _quantize(x, scale_fmt, None)
    return data, scales


def quantize_index_folded(x, weights, scale_fmt="ue8m0"):
    """``quantize_index(x)`` plus the indexer weight fold in the same pass.

    Returns ``(data, scales, folded)`` with ``folded = weights * scales[..., 0]``
    computed in fp32 by the quantiser (the fold of
    ``models/deepseek_v32/projections.py:241-244``). ``weights`` is FP32 with
    the shape ``x.shape[:-1]``.
    """
    if (
        not isinstance(weights, torch.Tensor)
        or weights.dtype != torch.float32
        or not isinstance(x, torch.Tensor)
        or tuple(weights.shape) != tuple(x.shape[:-1])
        or weights.device != x.device
    ):
        raise ValueError("weights must be FP32 with the shape of x without its last dimension")
    return _quantize(x, scale_fmt, weights)


def _quantize(x, scale_fmt, weights):
    if scale_fmt not in ("ue8m0", None):
        raise ValueError("Unsupported indexer quantization scale format")
    if not isinstance(x, torch.Tensor) or x.ndim == 0:
        raise ValueError("quantize_index expects a tensor with a last dimension")
    if x.dtype not in _native.DTYPE_CODES:
        raise ValueError("quantize_index supports bf16, fp16 and fp32 inputs")
    _native.require_gfx950(x.device, "indexer quantization")
    dim = x.shape[-1]
    if dim == 0:
        raise ValueError("quantize_index needs a nonempty last dimension")
    data = torch.empty(x.shape, dtype=torch.float8_e4m3fn, device=x.device)
    scales = torch.empty((*x.shape[:-1], 1), dtype=torch.float32, device=x.device)
    folded = None
    if weights is not None:
        weights = weights.contiguous()
        folded = torch.empty_like(weights)
    rows = x.numel() // dim
    if rows == 0:
        return data, scales, folded
    # Rows must sit at a uniform stride with unit element stride; other
    # layouts are copied on the device first.
    if x.is_contiguous():
        source, row_stride = x, dim
    elif x.ndim == 2 and x.stride(1) == 1:
        source, row_stride = x, x.stride(0)
    else:
        source, row_stride = x.contiguous(), dim
    common = (
        _native.ptr(source),
        _native.DTYPE_CODES[x.dtype],
        rows,
        dim,
        row_stride,
        _native.ptr(data),
        _native.ptr(scales),
        1 if scale_fmt == "ue8m0" else 0,
    )
    with torch.cuda.device(x.device):
        if weights is None:
            _native.call("dsa_quantize_fp8_rows", *common, _native.stream_of(x.device))
        else:
            _native.call("dsa_quantize_fp8_rows_fold", *common, _native.ptr(weights),
                         _native.ptr(folded), _native.stream_of(x.device))
    return data, scales, folded


def quantize_into(x, codes, scales, scale_fmt="ue8m0"):
    """Quantise bf16/fp16/fp32 rows ``x [R, D]`` straight into preallocated
    storage: ``codes`` e4m3 ``[R, D]`` and ``scales`` fp32 ``[R]`` (both
    contiguous), e.g. a slice of the resident index-K cache
    (``models/deepseek_v32/attention.py:323-326``)."""
    if scale_fmt not in ("ue8m0", None):
        raise ValueError("Unsupported indexer quantization scale format")
    if x.ndim != 2 or x.dtype not in _native.DTYPE_CODES or x.stride(-1) != 1:
        raise ValueError("x must be [rows, dim] with a unit last-dim stride")
    rows, dim = x.shape
    if (codes.dtype != torch.float8_e4m3fn or tuple(codes.shape) != (rows, dim)
            or not codes.is_contiguous() or codes.device != x.device):
        raise ValueError("codes must be contiguous float8_e4m3fn [rows, dim] on the input device")
    if (scales.dtype != torch.float32 or scales.numel() != rows or not scales.is_contiguous()
            or scales.device != x.device):
        raise ValueError("scales must be contiguous float32 with one entry per row")
    _native.require_gfx950(x.device, "indexer quantization")
    if rows == 0:
        return codes, scales
    with torch.cuda.device(x.device):
        _native.call(
            "dsa_quantize_fp8_rows", _native.ptr(x), _native.DTYPE_CODES[x.dtype], rows, dim,
            x.stride(0), _native.ptr(codes), _native.ptr(scales),
            1 if scale_fmt == "ue8m0" else 0, _native.stream_of(x.device))
    return codes, scales


def padded_columns(columns):
    return (columns + SCORE_ALIGNMENT - 1) // SCORE_ALIGNMENT * SCORE_ALIGNMENT


def logits(q, k, weights, kscale, query_start, prefetch=None, *, _bounds=None,
           _pad_to_stride=False, _q_fold=None):
    """Return causal FP32 ``[Q,N]`` logits with a padded physical row stride.

    ``out[i, j] = kscale[j] * sum_h weights[i, h] * relu(q[i, h] . k[j])`` for
    ``starts[i] <= j < ends[i]`` and ``-inf`` elsewhere; the default bounds are
    ``[0, query_start + i + 1)``. Storage is ``[Q, ceil(N/256)*256]`` with every
    padded column ``-inf``; ``_pad_to_stride`` returns that whole contiguous
    matrix, otherwise the logical ``[Q, N]`` view of it (``echo.py:318-322``).

    ``prefetch`` must be ``None``: the reference's fused ECHO prefetch is
    replaced in this build by the top-k-driven gather (``token_pool``).
    ``_q_fold`` (f32 ``[Q, 4, 128]``, from the layer prologue) carries the
    partial folded queries the kernel would otherwise form; same result bits.
    """
    if type(_pad_to_stride) is not bool:
        raise ValueError("_pad_to_stride must be boolean")
    if prefetch is not None:
        raise NotImplementedError(
            "fused ECHO prefetch is replaced by the top-k-driven gather (token_pool)"
        )
    args, q_fold, output, _operands = _logits_launch_args(q, k, weights, kscale, query_start,
                                                          _bounds, _q_fold)
    device = q.device
    with torch.cuda.device(device):
        if q_fold is None:
            _native.call("dsa_indexer_logits_fp8", *args, _native.ptr(output),
                         _native.stream_of(device))
        else:
            _native.call("dsa_indexer_logits_fp8_folded", *args, _native.ptr(q_fold),
                         _native.ptr(output), _native.stream_of(device))
    return output if _pad_to_stride else output[:, :len(k)]


def logits_topk(q, k, weights, kscale, query_start, topk, *, _bounds=None, _q_fold=None):
    """``logits`` then ``exact_topk`` of its logical ``[Q, N]`` view, fused.

    The logits kernel also counts each row's scores by the top 11 bits of their
    radix key, and the top-k starts from those counts instead of its own
    histogram pass over the scores (the coarse score buckets of the reference's
    fused ECHO kernel, ``indexer/csrc/echo_logits.cuh:497-561``, put to the
    selection instead of the prefetch). Returns ``(scores, values, indices)``:
    the padded score matrix of ``logits(..., _pad_to_stride=True)`` and the
    ``exact_topk(scores[:, :N], topk)`` outputs, bit for bit the unfused ones.
    This is the indexer step of ``models/deepseek_v32/attention.py:338-363``.
    """
    if type(topk) is not int or not 1 <= topk <= 2048:
        raise ValueError("k must be an integer in [1, 2048]")
    args, q_fold, scores, _operands = _logits_launch_args(q, k, weights, kscale, query_start,
                                                          _bounds, _q_fold)
    rows, columns, device = len(q), len(k), q.device
    count = min(topk, columns)
    values = torch.empty((rows, count), dtype=torch.float32, device=device)
    indices = torch.empty((rows, count), dtype=torch.int32, device=device)
    with torch.cuda.device(device):
        stream = _native.stream_of(device)
        workspace = _digit_workspace(device, stream, rows, columns)
        _native.call("dsa_indexer_topk_fp8", *args, _native.ptr(q_fold), _native.ptr(scores), topk,
                     _native.ptr(values), _native.ptr(indices), count, _native.ptr(workspace),
                     workspace.numel(), stream)
    return scores, values, indices


def select_topk(q, k, weights, kscale, query_start, topk, *, _bounds=None, _q_fold=None,
                _list_cap=0, _floors=None, _floors_ready=False):
    """The indexer step's top-k without the score matrix: ``(values, indices)``
    equal, bit for bit, to ``exact_topk(logits(q, k, weights, kscale,
    query_start), topk)`` for every input.

    Three launches (``dsa_indexer_select_fp8``): per-row floors estimated from
    ~1/64 of each row's scores; the logits kernel writing only the composite
    top-k keys of the scores at or above the floor (per key split, ~4K per
    row at 64K keys, instead of every score); the exact top-k of those
    candidates, which raises a row's floor when it holds more candidates
    than its sort takes (8,192) and recomputes a row in full when it holds
    fewer than ``min(topk, N)`` of them. This replaces the reference's ``logits`` then
    ``exact_topk`` (``models/deepseek_v32/attention.py:338-363``); the
    per-query score buckets of its fused ECHO kernel play the same role
    (``indexer/csrc/echo_logits.cuh:497-561``).

    ``_floors_ready``: the floors are already in this stream's workspace
    (``select_floors_buffer``; the layer prologue writes them), so the
    floors launch is skipped. ``_list_cap`` (candidate slots per row and key
    split, 0 = default) and ``_floors`` (uint32 ``[Q]`` radix keys replacing
    the estimated floors, as int32) are test hooks: small lists force
    spills, high floors force the recompute and low ones the raised floor.
    """
    if type(topk) is not int or not 1 <= topk <= 2048:
        raise ValueError("k must be an integer in [1, 2048]")
    args, q_fold, _, _operands = _logits_launch_args(q, k, weights, kscale, query_start, _bounds,
                                                     _q_fold, allocate_output=False)
    rows, columns, device = len(q), len(k), q.device
    count = min(topk, columns)
    values = torch.empty((rows, count), dtype=torch.float32, device=device)
    indices = torch.empty((rows, count), dtype=torch.int32, device=device)
    head = args[:9]  # q, k, weights, kscale, starts, ends, query_start, rows, columns
    with torch.cuda.device(device):
        stream = _native.stream_of(device)
        workspace, scores = _select_buffers(device, stream, rows, columns, _list_cap)
        if _floors is None and _list_cap == 0 and not _floors_ready:
            _native.call("dsa_indexer_select_fp8", *head, _native.ptr(q_fold), _native.ptr(scores),
                         topk, _native.ptr(values), _native.ptr(indices), count,
                         _native.ptr(workspace), workspace.numel(), stream)
            return values, indices
        floors = workspace[:8 * rows].view(torch.int32).view(rows, 2)
        if not _floors_ready:
            _native.call("dsa_indexer_floors_fp8", *head, topk, _native.ptr(floors), stream)
        if _floors is not None:
            _check_tensor(_floors, (rows,), torch.int32, device, "_floors")
            floors.copy_(_floors[:, None].expand(rows, 2))
        _native.call("dsa_indexer_logits_fp8_emit", *head, scores.shape[1], _native.ptr(q_fold),
                     _native.ptr(scores), _list_cap, _native.ptr(workspace), workspace.numel(),
                     stream)
        _native.call("dsa_indexer_emit_topk", *head, _native.ptr(q_fold), _native.ptr(scores), topk,
                     _native.ptr(values), _native.ptr(indices), count, _list_cap,
                     _native.ptr(workspace), workspace.numel(), stream)
    return values, indices


def select_floors_buffer(device, rows, columns):
    """The floors (int32 ``[rows, 2]``: two estimates per row, the row's floor
    being the smaller as uint32) of the current stream's ``select_topk``
    workspace for ``rows`` x ``columns``: a producer that computes the floors
    itself (``dsa_layer_prologue_floors_fp8``) writes them here, then calls
    ``select_topk(..., _floors_ready=True)``."""
    with torch.cuda.device(device):
        workspace, _ = _select_buffers(device, _native.stream_of(device), rows, columns, 0)
    return workspace[:8 * rows].view(torch.int32).view(rows, 2)


def select_floors(q, k, weights, kscale, query_start, topk, *, _bounds=None):
    """The per-row floors ``select_topk`` estimates (uint32 radix keys as
    int32 ``[Q]``; 0 for rows selected from their full scores)."""
    args, _, _, _operands = _logits_launch_args(q, k, weights, kscale, query_start, _bounds, None,
                                                allocate_output=False)
    floors = torch.empty((len(q), 2), dtype=torch.int32, device=q.device)
    with torch.cuda.device(q.device):
        _native.call("dsa_indexer_floors_fp8", *args[:9], topk, _native.ptr(floors),
                     _native.stream_of(q.device))
    return floors[:, 0].contiguous()


def _logits_launch_args(q, k, weights, kscale, query_start, bounds, q_fold, allocate_output=True):
    """Validation of ``echo.py:299-330`` and the kernel arguments up to ``ldo``;
    returns ``(args, q_fold, output, operands)`` with the padded output
    allocated (None with ``allocate_output=False``); ``operands`` holds the
    (possibly realigned) inputs the pointers in ``args`` refer to, to be kept
    alive until the launch."""
    if q.ndim != 3 or q.shape[1:] != (64, 128) or not q.is_cuda or len(q) < 1:
        raise ValueError("ECHO requires nonempty CUDA Q[query,64,128]")
    if k.ndim != 2 or k.shape[1] != 128 or len(k) < 1:
        raise ValueError("ECHO requires nonempty K[token,128]")
    rows, columns, device = len(q), len(k), q.device
    if type(query_start) is not int or not 0 <= query_start <= columns - rows:
        raise ValueError("query_start must place all query rows inside the visible KV sequence")
    _native.require_gfx950(device, "fp8 MQA logits")
    for tensor, shape, dtype, name in (
        (q, (rows, 64, 128), torch.float8_e4m3fn, "q"),
        (k, (columns, 128), torch.float8_e4m3fn, "k"),
        (weights, (rows, 64), torch.float32, "weights"),
        (kscale, (columns,), torch.float32, "kscale"),
    ):
        _check_tensor(tensor, shape, dtype, device, name)
    starts = ends = None
    if bounds is not None:
        starts, ends = bounds
        _check_tensor(starts, (rows,), torch.int32, device, "starts")
        _check_tensor(ends, (rows,), torch.int32, device, "ends")
    if q_fold is not None:
        _check_tensor(q_fold, (rows, 4, 128), torch.float32, device, "_q_fold")
        if q_fold.data_ptr() % 16:
            q_fold = q_fold.clone()
    # The kernel reads q, k and weights in 16-byte units.
    q, k, weights = (t if t.data_ptr() % 16 == 0 else t.clone() for t in (q, k, weights))
    width = padded_columns(columns)
    output = (torch.empty((rows, width), dtype=torch.float32, device=device)
              if allocate_output else None)
    args = [_native.ptr(q), _native.ptr(k), _native.ptr(weights), _native.ptr(kscale),
            _native.ptr(starts), _native.ptr(ends), query_start, rows, columns, width]
    return args, q_fold, output, (q, k, weights)


def exact_topk(scores, k):
    """Return descending values and int32 token IDs; nonfinite slots use -1.

    ``scores`` is FP32 ``[query, visible_tokens]`` (any row stride, unit column
    stride preferred). Order is descending by the fp32 radix key (``-0.0`` below
    ``+0.0``), ties to the smaller index (SMALL), matching FlashInfer's
    deterministic radix top-k with the reference's mask (``selection.py:62-113``).
    Capacity is ``min(k, visible_tokens)``.
    """
    if (
        not isinstance(scores, torch.Tensor)
        or scores.ndim != 2
        or scores.shape[1] < 1
        or scores.dtype != torch.float32
        or scores.requires_grad
    ):
        raise ValueError("scores must be inference FP32 [query, nonempty visible_tokens]")
    if type(k) is not int or not 1 <= k <= 2048:
        raise ValueError("k must be an integer in [1, 2048]")
    if not scores.is_cuda:
        raise NotImplementedError("DSA exact selection requires an MI355X (gfx950) HIP device")
    _native.require_gfx950(scores.device, "DSA exact selection")
    rows, columns = scores.shape
    count = min(k, columns)
    device = scores.device
    values = torch.empty((rows, count), dtype=torch.float32, device=device)
    indices = torch.empty((rows, count), dtype=torch.int32, device=device)
    if rows == 0:
        return values, indices
    if scores.stride(1) != 1 or scores.stride(0) < columns:
        scores = scores.contiguous()
    with torch.cuda.device(device):
        stream = _native.stream_of(device)
        workspace = _topk_workspace(device, stream, rows)
        _native.call(
            "dsa_topk_radix_split",
            _native.ptr(scores),
            rows,
            columns,
            scores.stride(0),
            k,
            _native.ptr(values),
            _native.ptr(indices),
            count,
            _native.ptr(workspace),
            workspace.numel(),
            stream,
        )
    return values, indices


# Per (device, stream) workspace of the two-part top-k (the sorted half lists
# of every row), reused by all stream-ordered calls on that stream.
_TOPK_WORKSPACES = {}

# Per (device, stream) workspace of ``logits_topk`` (radix-digit counts, list
# fill and key lists) and the row count of its last call: zero-filled when
# allocated; every fused call leaves the counts and fill of its layout zero.
_DIGIT_WORKSPACES = {}


def _digit_workspace(device, stream, rows, columns):
    """The (device, stream) workspace of the fused indexer step. Its layout
    depends on the row count, and a call only restores the zeros of its own
    layout, so a call with another row count zeroes it first."""
    key = (device.index, stream.value)
    workspace, layout_rows = _DIGIT_WORKSPACES.get(key, (None, None))
    needed = ctypes.c_int64()
    _native.call("dsa_indexer_topk_workspace_bytes", rows, columns, ctypes.byref(needed))
    if workspace is None or workspace.numel() < needed.value:
        workspace = torch.zeros(needed.value, dtype=torch.uint8, device=device)
    elif layout_rows != rows:
        workspace.zero_()
    _DIGIT_WORKSPACES[key] = (workspace, rows)
    return workspace


# Per (device, stream) workspace and score scratch of ``select_topk``: the
# workspace needs no initialisation; the scratch holds rows stored in full and
# spilled columns.
_SELECT_BUFFERS = {}


def _select_buffers(device, stream, rows, columns, list_cap):
    key = (device.index, stream.value)
    workspace, scores = _SELECT_BUFFERS.get(key, (None, None))
    needed = ctypes.c_int64()
    _native.call("dsa_indexer_select_workspace_bytes", rows, columns, list_cap,
                 ctypes.byref(needed))
    if workspace is None or workspace.numel() < needed.value:
        # 256-byte alignment: the caching allocator's blocks are 512-aligned.
        workspace = torch.empty(needed.value, dtype=torch.uint8, device=device)
    width = padded_columns(columns)
    if scores is None or scores.numel() < rows * width:
        scores = torch.empty(rows * width, dtype=torch.float32, device=device)
    _SELECT_BUFFERS[key] = (workspace, scores)
    return workspace, scores[:rows * width].view(rows, width)


def _topk_workspace(device, stream, rows):
    key = (device.index, stream.value)
    workspace = _TOPK_WORKSPACES.get(key)
    needed = ctypes.c_int64()
    _native.call("dsa_topk_workspace_bytes", rows, ctypes.byref(needed))
    if workspace is None or workspace.numel() < needed.value:
        workspace = torch.empty(needed.value, dtype=torch.uint8, device=device)
        _TOPK_WORKSPACES[key] = workspace
    return workspace
