"""A7: sparse MLA over selected token records (TEST INFRASTRUCTURE ONLY).

Restates ``reference_sparse_mla``
(``operators/deepseek_v32/attention/reference/torch.py:13-28``): for each
query row, the selected ids in ``[0, N)`` address KV records (duplicates count
once per slot, negative or out-of-range ids are padding), and in fp32

    P = softmax_j(q[r] @ kv[S_r].T * scale)     out[r] = P @ kv[S_r, :value_dim]

rounded to bf16. A row without a valid id is all zeros. int64 ids are masked
before narrowing (``attention/device_only/mla.py:78-82``), which this oracle
gets for free by comparing in int64.

Pinned by ``tests/test_oracle_sparse_mla.py``: the reference's known answers
(duplicates/padding -> 4, 0, 2; RoPE dimensions only steer scores -> 0.75;
+-100 x 100 logits around empty tiles -> exactly 2; int64 ids that would wrap
when narrowed -> padding; empty inputs -> zeros), ``sparse_mla_brute_force``
(float64 scalar loops) on small random shapes with duplicates, padding and
out-of-range ids, and closed forms (one valid key -> its value row, equal
scores -> the mean value row). The same file plants mistakes in copies of
this function and requires the pins to catch each.
"""

import numpy as np

from oracle import fp8


def sparse_mla(q, kv, indices, scale, value_dim=512):
    """q float32 [Q,H,D], kv float32 [N,D], indices int [Q,K] -> bf16 bits [Q,H,value_dim].

    Returns the bf16 bit patterns (uint16) of the result and the float32 result
    before rounding, as a tuple.
    """
    q = np.asarray(q, dtype=np.float32)
    kv = np.asarray(kv, dtype=np.float32)
    indices = np.asarray(indices).astype(np.int64)
    rows, heads, _ = q.shape
    out = np.zeros((rows, heads, value_dim), dtype=np.float32)
    for r in range(rows):
        sel = indices[r]
        sel = sel[(sel >= 0) & (sel < kv.shape[0])]
        if not sel.size:
            continue
        records = kv[sel]
        logits = (q[r] @ records.T) * np.float32(scale)
        logits = logits - logits.max(axis=-1, keepdims=True)
        p = np.exp(logits)
        p /= p.sum(axis=-1, keepdims=True)
        out[r] = p @ records[:, :value_dim]
    return fp8.f32_to_bf16_bits(out), out


def sparse_mla_brute_force(q, kv, indices, scale, value_dim):
    """Float64 loops for small shapes (pins ``sparse_mla``)."""
    q = np.asarray(q, dtype=np.float64)
    kv = np.asarray(kv, dtype=np.float64)
    rows, heads, dim = q.shape
    out = np.zeros((rows, heads, value_dim))
    for r in range(rows):
        sel = [int(j) for j in indices[r] if 0 <= int(j) < kv.shape[0]]
        if not sel:
            continue
        for h in range(heads):
            s = [sum(q[r, h, d] * kv[j, d] for d in range(dim)) * scale for j in sel]
            m = max(s)
            e = [np.exp(x - m) for x in s]
            z = sum(e)
            for v in range(value_dim):
                out[r, h, v] = sum(e[t] * kv[sel[t], v] for t in range(len(sel))) / z
    return out
