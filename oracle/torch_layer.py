"""The DSA layer on torch's CPU kernels (TEST INFRASTRUCTURE ONLY).

The multi-threaded restatement of ``oracle.layer.dsa_layer`` that
``bench.py``'s ``cpu_baseline`` leg times: the same stages and arithmetic
(models/deepseek_v32/attention.py:276-425), with the per-stage formulas of
``oracle.quantize`` (A1), ``oracle.logits`` (A4), ``oracle.topk`` (A6) and
``oracle.sparse_mla`` (A7) written as torch tensor operations so that torch's
intra-op thread pool runs them on every core it is given:

* A1: per-row amax, ``max(amax, 1e-4) * fl32(1/448)`` rounded up to a power of
  two, ``x * (1 / scale)`` clamped to +-448 and cast to e4m3 (torch's
  ``float8_e4m3fn`` cast rounds to nearest even, as ``oracle.fp8.encode``);
* A4: ``kscale[j] * sum_h w[i, h] * relu(q[i, h] . k[j])`` on the decoded fp8
  values, ``-inf`` outside ``j < history + 1 + i`` and in the stride padding;
* A6: descending by the radix order of the fp32 bits, equal keys by the
  smaller column (one int64 composite key per score), ``-1`` ids for
  non-finite values;
* A7: softmax over the selected records (duplicates count per slot, padding
  ids skipped) in fp32, ``P @ V`` rounded to bf16.

Finite inputs only (the bench's synthetic data); NaN rules stay with the
numpy oracle. Pinned by ``tests/test_oracle_torch_layer.py`` against
``oracle.layer.dsa_layer`` on the same inputs: quantisation and top-k
bit-for-bit, scores to 2e-6 of the row's largest score (the BLAS calls may sum
in another order), ids equal to the oracle top-k of the same scores, outputs to
bf16 rounding.
"""

import numpy as np
import torch

RECIPROCAL_448 = float(np.float32(1.0) / np.float32(448.0))


def _ue8m0_scales(x):
    amax = x.abs().amax(dim=-1, keepdim=True).clamp_min(1e-4)
    scale = (amax * RECIPROCAL_448).to(torch.float32)
    bits = scale.view(torch.int32)
    return ((bits + 0x7FFFFF) & 0x7F800000).view(torch.float32)


def quantize_index(x):
    """float32 [..., D] -> (decoded e4m3 values float32 [..., D], scales [..., 1])."""
    scale = _ue8m0_scales(x)
    y = (x * (1.0 / scale)).clamp(-448.0, 448.0)
    return y.to(torch.float8_e4m3fn).to(torch.float32), scale


class HistoryCache:
    """Decoded resident caches of a layer's history (built once, as on the GPU)."""

    def __init__(self, index_k, records_f32):
        self.k, k_scale = quantize_index(index_k)
        self.k_scale = k_scale[:, 0].contiguous()
        self.kt = self.k.t().contiguous()
        self.records = records_f32.contiguous()


def index_scores(index_q, weights, cache, history, rows, chunk=8):
    """A1 (Q), A2, A4 for the absolute query rows ``rows``."""
    q, q_scale = quantize_index(index_q[rows])
    w = weights[rows] * q_scale[..., 0]
    columns = cache.k.shape[0]
    width = (columns + 255) // 256 * 256
    out = torch.full((len(rows), width), float("-inf"), dtype=torch.float32)
    positions = torch.arange(columns)
    ends = history + 1 + torch.as_tensor(rows)
    heads, dim = q.shape[1], q.shape[2]
    for start in range(0, len(rows), chunk):
        stop = min(len(rows), start + chunk)
        raw = (q[start:stop].reshape(-1, dim) @ cache.kt).clamp_min_(0.0)
        value = torch.bmm(w[start:stop].unsqueeze(1), raw.view(stop - start, heads, columns)).squeeze(1)
        value *= cache.k_scale
        visible = positions[None, :] < ends[start:stop, None]
        out[start:stop, :columns] = torch.where(visible, value, torch.tensor(float("-inf")))
    return out


def exact_topk(scores, k):
    """float32 [R, C] -> (values, ids int32); radix order, smaller column on ties."""
    count = min(k, scores.shape[1])
    bits = scores.contiguous().view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    keys = torch.where(bits >= 0x80000000, bits ^ 0xFFFFFFFF, bits | 0x80000000)
    columns = torch.arange(scores.shape[1], dtype=torch.int64)
    composite = (keys << 31) - columns  # keys < 2^32, columns < 2^31
    _, order = torch.topk(composite, count, dim=1, sorted=True)
    values = torch.gather(scores, 1, order)
    ids = order.to(torch.int32)
    ids[~torch.isfinite(values)] = -1
    return values, ids


def sparse_mla(q, records, ids, scale, value_dim=512):
    """q float32 [Q,H,D], records float32 [N,D], ids [Q,K] -> float32 [Q,H,value_dim] (bf16-rounded)."""
    rows, heads, _ = q.shape
    out = torch.zeros((rows, heads, value_dim), dtype=torch.float32)
    for r in range(rows):
        sel = ids[r].to(torch.int64)
        sel = sel[(sel >= 0) & (sel < records.shape[0])]
        if sel.numel() == 0:
            continue
        kv = records.index_select(0, sel)
        logits = (q[r] @ kv.t()) * scale
        p = torch.softmax(logits, dim=-1)
        out[r] = p @ kv[:, :value_dim]
    return out.to(torch.bfloat16).to(torch.float32)


def dsa_layer(index_q, weights, mla_q, cache, history, rows, k=2048, scale=576**-0.5):
    """Returns (scores, values, ids, out) for the query rows ``rows``."""
    scores = index_scores(index_q, weights, cache, history, rows)
    values, ids = exact_topk(scores, k)
    out = sparse_mla(mla_q[rows], cache.records, ids, scale)
    return scores, values, ids, out
