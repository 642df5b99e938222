"""CPU DSA layer: indexer -> exact top-k -> sparse MLA (TEST INFRASTRUCTURE ONLY).

The stage order of ``models/deepseek_v32/attention.py:276-425`` on the oracle
functions of this package. Used by the full-layer parity test and as the
``cpu_baseline`` leg of ``bench.py``. Pinned through the functions it
composes (each pinned in its own test module); the composition itself is
checked against the stage-by-stage GPU results in ``tests/test_gpu_layer.py``.
"""

import numpy as np

from oracle import fp8, kv_fp8, logits, quantize, sparse_mla, topk


def f32(t):
    return t.float().cpu().numpy() if hasattr(t, "float") else np.asarray(t, np.float32)


class HistoryCache:
    """Quantised resident caches of a layer's history (built once, like the GPU's)."""

    def __init__(self, index_k_f32, kv_bf16_bits, fp8_records=True):
        self.k_codes, k_scale = quantize.quantize_index(index_k_f32)
        self.k_scale = k_scale[:, 0]
        if fp8_records:
            self.records = kv_fp8.decode_records(kv_fp8.encode_records(kv_bf16_bits))
        else:
            self.records = fp8.bf16_bits_to_f32(kv_bf16_bits)


def index_scores(index_q_f32, weights, cache, history, rows):
    """A1 (Q), A2, A4 for the query rows ``rows`` (absolute query indices)."""
    q_codes, q_scale = quantize.quantize_index(index_q_f32[rows])
    w = (np.asarray(weights, np.float32)[rows] * q_scale[..., 0]).astype(np.float32)
    ends = history + 1 + np.asarray(rows)
    return logits.logits(q_codes, cache.k_codes, w, cache.k_scale, 0,
                         starts=np.zeros(len(rows), np.int64), ends=ends,
                         pad_to_stride=True)


def dsa_layer(index_q_f32, weights, mla_q_f32, cache, history, rows, k=2048,
              scale=576**-0.5):
    """Returns (scores, values, ids, out_f32) for the selected query rows."""
    scores = index_scores(index_q_f32, weights, cache, history, rows)
    values, ids = topk.exact_topk(scores, k)
    _, out = sparse_mla.sparse_mla(mla_q_f32[rows], cache.records, ids, scale)
    return scores, values, ids, out
