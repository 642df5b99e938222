"""A4: fp8 MQA indexer logits with the causal -inf tail (TEST INFRASTRUCTURE ONLY).

Restates the resident branch of ``logits`` in
``operators/deepseek_v32/indexer/echo.py:339-410`` through the fp32 oracle its
tests use (``indexer/tests/test_echo_indexer.py:102-106``):

    out[i, j] = kscale[j] * sum_h w[i, h] * relu(sum_d q[i, h, d] * k[j, d])

for ``starts[i] <= j < ends[i]`` and ``-inf`` elsewhere, with
``ends[i] = query_start + i + 1`` and ``starts[i] = 0`` by default
(``echo.py:357-361``). The output row stride is ``ceil(N / 256) * 256``; the
padded columns are ``-inf`` (``echo.py:381,397-409``).

Pinned by ``tests/test_oracle_logits_topk.py``: a float64 brute-force loop on tiny
shapes, closed forms (zero weights give exactly 0, a one-hot head weight gives
``relu(q_h . k) * kscale``, all-negative dot products give 0) and the exact
``-inf`` placement for every causal boundary of a small case.
"""

import numpy as np

from oracle import fp8


def padded_width(columns):
    return (columns + 255) // 256 * 256


def logits(q_codes, k_codes, weights, kscale, query_start, *, starts=None, ends=None,
           pad_to_stride=False, chunk=16):
    """q_codes uint8 [Q,64,128], k_codes uint8 [N,128] -> float32 [Q, N or padded]."""
    q = fp8.decode(q_codes)
    k = fp8.decode(k_codes)
    rows, heads, dim = q.shape
    columns = k.shape[0]
    weights = np.asarray(weights, dtype=np.float32)
    kscale = np.asarray(kscale, dtype=np.float32)
    if ends is None:
        ends = query_start + 1 + np.arange(rows, dtype=np.int64)
    if starts is None:
        starts = np.zeros(rows, dtype=np.int64)
    width = padded_width(columns) if pad_to_stride else columns
    out = np.full((rows, width), -np.inf, dtype=np.float32)
    positions = np.arange(columns)
    kt = np.ascontiguousarray(k.T)
    for start in range(0, rows, chunk):
        stop = min(rows, start + chunk)
        raw = q[start:stop].reshape(-1, dim) @ kt  # [(rows*heads), N]
        np.maximum(raw, 0, out=raw)
        raw = raw.reshape(stop - start, heads, columns)
        value = np.einsum("qhn,qh->qn", raw, weights[start:stop], optimize=True)
        value *= kscale[None, :]
        visible = (positions[None, :] >= np.asarray(starts[start:stop])[:, None]) & (
            positions[None, :] < np.asarray(ends[start:stop])[:, None]
        )
        out[start:stop, :columns] = np.where(visible, value, -np.inf)
    return out


def logits_brute_force(q_codes, k_codes, weights, kscale, query_start):
    """Pure-Python float64 loops; only for tiny shapes (pins ``logits``)."""
    q = fp8.decode(q_codes).astype(np.float64)
    k = fp8.decode(k_codes).astype(np.float64)
    rows, heads, dim = q.shape
    columns = k.shape[0]
    out = [[float("-inf")] * columns for _ in range(rows)]
    for i in range(rows):
        for j in range(min(columns, query_start + i + 1)):
            total = 0.0
            for h in range(heads):
                dot = 0.0
                for d in range(dim):
                    dot += q[i, h, d] * k[j, d]
                total += float(weights[i][h]) * max(dot, 0.0)
            out[i][j] = total * float(kscale[j])
    return np.array(out, dtype=np.float64)
