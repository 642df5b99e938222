"""Sparse MLA prefill on MI355X over bf16 records or the fp8 paged KV cache.

Drop-in for the reference's attention operators (same names, argument order,
padding semantics and validation messages):

* ``sparse_mla``           - ``operators/deepseek_v32/attention/device_only/mla.py:90-115``
  with ``_validate`` (``attention/_validation.py:8-24``) and the input
  preparation of ``mla.py:70-87`` (contiguity, 16-byte alignment, int64 ids
  masked before narrowing). The selection is not padded to 128: the kernel
  accepts any count.
* ``sparse_mla_from_pool`` - ``operators/deepseek_v32/attention/offload/mla.py:12-20``.
* ``sparse_mla_fp8_paged`` - the same attention over the 656-byte fp8 paged
  record (512 e4m3 + 4 fp32 tile scales + 64 bf16 RoPE, 64 tokens per page),
  which has no reference counterpart.
* ``pack_kv_fp8``          - writes bf16 ``[T, 576]`` records into that cache
  (quantise-on-append).

Kernels: ``csrc/sparse_mla.hip`` and ``csrc/quantize.hip``.
"""

import math

import torch

from cxldsagr_amd import _native

QK_DIM = 576
V_DIM = 512
PAGE_TOKENS = 64
RECORD_BYTES = 656


def _validate(q, kv, indices, scale, value_dim):
    """Mirror of ``attention/_validation.py:8-24``."""
    if q.ndim != 3 or kv.ndim != 2 or indices.ndim != 2:
        raise ValueError("Expected q [Q,H,D], kv [N,D], and indices [Q,K]")
    if q.shape[0] != indices.shape[0] or q.shape[-1] != kv.shape[-1]:
        raise ValueError("Query, cache, and selection dimensions do not agree")
    if not isinstance(value_dim, int) or not 1 <= value_dim <= q.shape[-1]:
        raise ValueError("value_dim must be an integer in [1, query dimension]")
    if value_dim > 512 or q.shape[-1] - value_dim > 128:
        raise ValueError("Supported dimensions are value_dim <= 512 and position dimension <= 128")
    if q.device != kv.device or q.device != indices.device:
        raise ValueError("q, kv, and indices must be on the same device")
    if q.dtype != kv.dtype or not q.is_floating_point():
        raise ValueError("q and kv must share a floating-point dtype")
    if indices.dtype not in (torch.int32, torch.int64):
        raise ValueError("indices must be int32 or int64")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")


def _check_layout(q, value_dim, what):
    _native.require_gfx950(q.device, what)
    if q.dtype != torch.bfloat16:
        raise ValueError("DSA sparse MLA requires BF16 queries and KV records")
    if q.shape[1] % 64 or q.shape[1] == 0 or q.shape[2] != QK_DIM or value_dim != V_DIM:
        raise ValueError("DeepSeek sparse MLA requires H a multiple of 64, QK dimension 576 and V=512")


def _aligned(tensor):
    tensor = tensor.contiguous()
    if tensor.data_ptr() % 16:
        tensor = tensor.clone()
    return tensor


def _narrow_ids(indices, limit):
    if indices.dtype == torch.int64:
        # Mask before narrowing so large invalid ids cannot wrap into valid ones.
        valid = (indices >= 0) & (indices < limit)
        indices = indices.masked_fill(~valid, -1).to(torch.int32)
    return indices.contiguous()


def sparse_mla(q, kv, indices, scale, value_dim=512):
    """Return BF16 ``[Q,H,512]`` sparse attention over bf16 ``kv [N,576]`` records.

    Negative and out-of-range ids are padding; duplicates participate
    independently; all-padding rows return zero. H may be any multiple of 64.
    """
    _validate(q, kv, indices, scale, value_dim)
    _check_layout(q, value_dim, "DSA sparse MLA")
    if kv.shape[0] > torch.iinfo(torch.int32).max:
        raise ValueError("sparse MLA requires the KV row count to fit int32")
    if not q.shape[0] or not kv.shape[0] or not indices.shape[1]:
        return torch.zeros((*q.shape[:2], value_dim), dtype=q.dtype, device=q.device)
    # The kernel writes every output element (all-padding rows as zeros).
    out = torch.empty((*q.shape[:2], value_dim), dtype=q.dtype, device=q.device)
    q, kv = _aligned(q), _aligned(kv)
    ids = _narrow_ids(indices, kv.shape[0])
    with torch.cuda.device(q.device):
        _native.call(
            "dsa_sparse_mla_bf16",
            _native.ptr(q), q.shape[0], q.shape[1],
            _native.ptr(kv), kv.shape[0],
            _native.ptr(ids), ids.shape[1],
            float(scale),
            _native.ptr(out),
            _native.stream_of(q.device),
        )
    return out


def sparse_mla_from_pool(q, records, physical_indices, scale, value_dim=512):
    """Consume recalled HBM records using physical pool ids (``offload/mla.py:12-20``).

    Every non-padding id must already name its selected record in ``records``;
    the caller keeps the selected slots resident until stream completion.
    """
    return sparse_mla(q, records, physical_indices, scale, value_dim)


def _check_paged(cache, page_table, device):
    if (
        not isinstance(cache, torch.Tensor)
        or cache.dtype != torch.uint8
        or cache.ndim != 3
        or cache.shape[1:] != (PAGE_TOKENS, RECORD_BYTES)
        or cache.device != device
    ):
        raise ValueError("kv_cache must be uint8 [pages, 64, 656] on the query device")
    if (
        not isinstance(page_table, torch.Tensor)
        or page_table.dtype != torch.int32
        or page_table.ndim != 1
        or page_table.device != device
    ):
        raise ValueError("page_table must be int32 [logical_pages] on the query device")


def sparse_mla_fp8_paged(q, kv_cache, page_table, indices, scale, value_dim=512, *,
                         n_tokens=None, _out=None):
    """Sparse MLA over the fp8 paged cache; same semantics as ``sparse_mla`` on the
    dequantised records.

    ``kv_cache`` is uint8 ``[pages, 64, 656]``; logical token ``t`` lives at
    page ``page_table[t // 64]``, slot ``t % 64``. Ids outside ``[0, n_tokens)``
    (default: every token the page table covers) are padding. ``_out``
    (contiguous, ``q``'s dtype and device, ``[Q, H, value_dim]``) receives the
    result instead of a new tensor.
    """
    if q.ndim != 3 or indices.ndim != 2 or q.shape[0] != indices.shape[0]:
        raise ValueError("Expected q [Q,H,D] and indices [Q,K] with matching Q")
    if indices.dtype not in (torch.int32, torch.int64) or indices.device != q.device:
        raise ValueError("indices must be int32 or int64 on the query device")
    if not math.isfinite(scale):
        raise ValueError("scale must be finite")
    _check_layout(q, value_dim, "DSA fp8 paged sparse MLA")
    _check_paged(kv_cache, page_table, q.device)
    if n_tokens is None:
        n_tokens = page_table.numel() * PAGE_TOKENS
    if type(n_tokens) is not int or not 0 <= n_tokens <= page_table.numel() * PAGE_TOKENS:
        raise ValueError("n_tokens must be covered by the page table")
    shape = (*q.shape[:2], value_dim)
    if _out is None:
        out = torch.empty(shape, dtype=q.dtype, device=q.device)
    elif (not isinstance(_out, torch.Tensor) or tuple(_out.shape) != shape or _out.dtype != q.dtype
          or _out.device != q.device or not _out.is_contiguous()
          or _out.data_ptr() % 8):
        raise ValueError("_out must be a contiguous, 8-byte aligned [Q, H, value_dim] tensor "
                         "of q's dtype on q's device")
    else:
        out = _out
    if not q.shape[0] or not n_tokens or not indices.shape[1]:
        return out.zero_()
    q = _aligned(q)
    cache = _aligned(kv_cache)
    table = page_table.contiguous()
    ids = _narrow_ids(indices, n_tokens)
    with torch.cuda.device(q.device):
        _native.call(
            "dsa_sparse_mla_fp8_paged",
            _native.ptr(q), q.shape[0], q.shape[1],
            _native.ptr(cache), cache.shape[0],
            _native.ptr(table), n_tokens,
            _native.ptr(ids), ids.shape[1],
            float(scale),
            _native.ptr(out),
            _native.stream_of(q.device),
        )
    return out


def pack_kv_fp8(kv, kv_cache, page_table, token_offset=0, status=None):
    """Quantise bf16 ``kv [T, 576]`` into the fp8 paged cache at tokens
    ``token_offset .. token_offset + T`` (A1 rule per 128-value latent tile,
    UE8M0 scales, RoPE copied). ``status`` (int32 [1], optional) gets bit 0 set
    if a page number lies outside the cache.
    """
    if kv.ndim != 2 or kv.shape[1] != QK_DIM or kv.dtype != torch.bfloat16:
        raise ValueError("kv must be bf16 [tokens, 576]")
    _native.require_gfx950(kv.device, "fp8 KV pack")
    _check_paged(kv_cache, page_table, kv.device)
    if not kv_cache.is_contiguous():
        raise ValueError("kv_cache must be contiguous")
    tokens = kv.shape[0]
    if type(token_offset) is not int or token_offset < 0:
        raise ValueError("token_offset must be a nonnegative integer")
    if token_offset + tokens > page_table.numel() * PAGE_TOKENS:
        raise ValueError("tokens exceed the pages covered by the page table")
    if status is not None and (status.dtype != torch.int32 or status.device != kv.device):
        raise ValueError("status must be int32 on the cache device")
    if tokens == 0:
        return kv_cache
    kv = _aligned(kv)
    if kv_cache.data_ptr() % 16:
        raise ValueError("kv_cache must be 16-byte aligned")
    with torch.cuda.device(kv.device):
        _native.call(
            "dsa_kv_pack_fp8",
            _native.ptr(kv), tokens, token_offset,
            _native.ptr(page_table.contiguous()), kv_cache.shape[0],
            _native.ptr(kv_cache),
            _native.ptr(status),
            _native.stream_of(kv.device),
        )
    return kv_cache
