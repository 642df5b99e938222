"""A6: exact top-k with SMALL tie order and -1 for non-finite (TEST INFRASTRUCTURE ONLY).

Restates ``exact_topk`` (``operators/deepseek_v32/indexer/selection.py:62-113``):
FlashInfer ``radix_topk`` in sorted, deterministic, ``TopKTieBreak.SMALL`` mode
followed by the non-finite index mask (``selection.py:43-51``).

* ``count = min(k, columns)``; ``1 <= k <= 2048``.
* Order: descending by the radix key of the fp32 bits (sign bit set: all bits
  flipped; else sign bit flipped), so ``-0.0`` ranks just below ``+0.0``;
  equal keys keep the smaller column first (SMALL). This is the composite
  ``(~ordered(value) << 32) | id`` order the reference spells out for its Q1
  path (``indexer/csrc/q1_topk_sort.cu:24-42``).
* Values keep their bits; the index is ``-1`` where ``|value|`` is inf or NaN.

Pinned by ``tests/test_oracle_logits_topk.py``: values equal ``torch.topk`` bit-for-bit,
ids equal torch's stable descending argsort on rows without signed zeros, the
reference's known answers (all-equal rows -> ``arange``, masked rows -> -1, the
signed-zero/extreme-value row), and a brute-force Python sort on small rows.

``digit_counts`` is the level-0 histogram of a radix selection over these keys
(per row, the count of keys by their top 11 bits): what FlashInfer's radix
top-k histograms first and, at a coarser width, the per-query score buckets
of the reference's ECHO logits kernel (``indexer/csrc/echo_logits.cuh:497-561``).
Pinned by the same test file: counts sum to the columns, a per-element Python
loop on small rows, and the bucket where the descending suffix count first
reaches ``k`` holds the ``k``-th value of ``exact_topk``.
"""

import numpy as np


def radix_keys(scores):
    """float32 array -> uint32 keys whose unsigned order is the float order."""
    bits = np.ascontiguousarray(scores, dtype=np.float32).view(np.uint32)
    negative = (bits >> 31) == 1
    return np.where(negative, ~bits, bits | np.uint32(0x80000000)).astype(np.uint32)


def exact_topk(scores, k):
    """float32 [R, C] -> (values float32 [R, c], ids int32 [R, c]), c = min(k, C)."""
    scores = np.asarray(scores, dtype=np.float32)
    if scores.ndim != 2 or scores.shape[1] < 1:
        raise ValueError("scores must be inference FP32 [query, nonempty visible_tokens]")
    if type(k) is not int or not 1 <= k <= 2048:
        raise ValueError("k must be an integer in [1, 2048]")
    rows, columns = scores.shape
    count = min(k, columns)
    keys = radix_keys(scores)
    # Stable sort on the complemented key: descending key, ascending column.
    order = np.argsort(~keys, axis=1, kind="stable")[:, :count]
    values = np.take_along_axis(scores, order, axis=1)
    ids = order.astype(np.int32)
    ids[~np.isfinite(values)] = -1
    return values, ids


DIGIT_BITS = 11


def digit_counts(scores):
    """float32 [R, C] -> int64 [R, 2048]: per row, keys by ``radix_key >> 21``."""
    keys = radix_keys(np.asarray(scores, dtype=np.float32)) >> np.uint32(32 - DIGIT_BITS)
    rows = keys.shape[0]
    counts = np.zeros((rows, 1 << DIGIT_BITS), dtype=np.int64)
    for r in range(rows):
        counts[r] = np.bincount(keys[r].astype(np.int64), minlength=1 << DIGIT_BITS)
    return counts
