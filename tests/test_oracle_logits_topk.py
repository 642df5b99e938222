"""Pins of the oracle's A4 logits and A6 top-k (CPU only).

Logits: float64 brute force on tiny shapes and closed forms
(operators/deepseek_v32/indexer/tests/test_echo_indexer.py:86-109,248-255).
Top-k: torch.topk values, torch's stable descending argsort, and the
reference's known answers (indexer/tests/test_selection.py:136-218).
"""

import numpy as np
import pytest
import torch

from oracle import fp8, logits, topk


def _codes(shape, rng, scale=1.0):
    return fp8.encode((rng.standard_normal(shape) * scale).astype(np.float32))


@pytest.mark.parametrize("rows,columns,query_start", [(1, 5, 4), (3, 9, 2), (4, 7, 3), (2, 2, 0)])
def test_logits_match_float64_brute_force(rows, columns, query_start):
    rng = np.random.default_rng(rows * 100 + columns)
    q = _codes((rows, 64, 128), rng)
    k = _codes((columns, 128), rng)
    w = (rng.standard_normal((rows, 64)) / 64).astype(np.float32)
    s = (rng.random(columns) + 0.5).astype(np.float32)
    ours = logits.logits(q, k, w, s, query_start)
    brute = logits.logits_brute_force(q, k, w, s, query_start)
    assert np.array_equal(np.isneginf(ours), np.isneginf(brute))
    finite = np.isfinite(brute)
    np.testing.assert_allclose(ours[finite], brute[finite], rtol=1e-5, atol=1e-5)


def test_logits_closed_forms():
    rng = np.random.default_rng(7)
    rows, columns = 3, 40
    q = _codes((rows, 64, 128), rng)
    k = _codes((columns, 128), rng)
    s = (rng.random(columns) + 0.5).astype(np.float32)
    # zero weights -> exactly zero on the visible prefix, -inf after it
    out = logits.logits(q, k, np.zeros((rows, 64), np.float32), s, columns - rows)
    ends = columns - rows + 1 + np.arange(rows)
    visible = np.arange(columns)[None] < ends[:, None]
    assert (out[visible] == 0).all() and np.isneginf(out[~visible]).all()
    # one-hot head weight -> relu(q_h . k) * kscale
    w = np.zeros((rows, 64), np.float32)
    w[:, 5] = 1.0
    out = logits.logits(q, k, w, s, columns - rows)
    qf, kf = fp8.decode(q).astype(np.float64), fp8.decode(k).astype(np.float64)
    expected = np.maximum(qf[:, 5] @ kf.T, 0) * s
    np.testing.assert_allclose(out[visible], expected[visible], rtol=1e-5, atol=1e-4)
    # all dot products negative -> relu kills every head -> exactly 0
    kneg = fp8.encode(-np.abs(fp8.decode(k)))
    qpos = fp8.encode(np.abs(fp8.decode(q)))
    out = logits.logits(qpos, kneg, np.ones((rows, 64), np.float32), s, columns - rows)
    assert (out[visible] == 0).all()


def test_logits_padded_width_and_bounds():
    rng = np.random.default_rng(3)
    q = _codes((2, 64, 128), rng)
    k = _codes((300, 128), rng)
    w = np.ones((2, 64), np.float32)
    s = np.ones(300, np.float32)
    out = logits.logits(q, k, w, s, 298, pad_to_stride=True)
    assert out.shape == (2, 512) and np.isneginf(out[:, 300:]).all()
    out = logits.logits(q, k, w, s, 0, starts=np.array([5, 0]), ends=np.array([10, 300]))
    assert np.isneginf(out[0, :5]).all() and np.isfinite(out[0, 5:10]).all()
    assert np.isneginf(out[0, 10:]).all() and np.isfinite(out[1]).all()


def test_radix_keys_order_like_floats_with_signed_zero():
    x = np.array([-np.inf, -3.0, -0.0, 0.0, 1e-30, 2.0, np.inf], np.float32)
    keys = topk.radix_keys(x)
    assert (np.diff(keys.astype(np.int64)) > 0).all()


@pytest.mark.parametrize("rows,columns,k", [(1, 1, 1), (3, 17, 2048), (5, 257, 32), (8, 4099, 1024)])
def test_topk_values_equal_torch_and_ids_equal_stable_argsort(rows, columns, k):
    gen = torch.Generator().manual_seed(191)
    scores = torch.randn(rows, columns, generator=gen)
    start = max(0, columns - rows)
    ends = (start + torch.arange(rows) + 1).clamp_max(columns)
    scores.masked_fill_(torch.arange(columns)[None] >= ends[:, None], -torch.inf)
    values, ids = topk.exact_topk(scores.numpy(), k)
    ref = scores.topk(min(k, columns), dim=-1)
    np.testing.assert_array_equal(values, ref.values.numpy())
    order = torch.argsort(scores, dim=-1, descending=True, stable=True)[:, : min(k, columns)]
    expected = order.int().masked_fill(~torch.isfinite(scores.gather(-1, order)), -1)
    np.testing.assert_array_equal(ids, expected.numpy())


def test_topk_small_ties_every_k_like_reference():
    scores = -torch.arange(2049, dtype=torch.float32).remainder(19)
    scores = scores.expand(3, -1).clone()
    scores[1].fill_(-torch.inf)
    scores[2, 31:] = -torch.inf
    reference_ids = torch.argsort(scores, dim=-1, descending=True, stable=True)
    reference_values = scores.gather(-1, reference_ids)
    for k in (1, 5, 19, 20, 107, 108, 1000, 2048):
        values, ids = topk.exact_topk(scores.numpy(), k)
        expected = reference_ids[:, :k].int().masked_fill(
            ~torch.isfinite(reference_values[:, :k]), -1)
        np.testing.assert_array_equal(ids, expected.numpy())
        np.testing.assert_array_equal(values, reference_values[:, :k].numpy())


def test_topk_known_answers():
    scores = np.zeros((3, 66560), np.float32)
    scores[1] = -np.inf
    scores[2, 7:] = -np.inf
    values, ids = topk.exact_topk(scores, 2048)
    assert (ids[0] == np.arange(2048)).all()
    assert (ids[1] == -1).all() and np.isneginf(values[1]).all()
    assert (ids[2, :7] == np.arange(7)).all() and (ids[2, 7:] == -1).all()
    row = np.array([[-0.0, 0.0, -0.0, 0.0, 1.0, -1.0, np.nan]], np.float32)
    values, ids = topk.exact_topk(row, 7)
    assert ids.tolist() == [[-1, 4, 1, 3, 0, 2, 5]]  # +NaN ranks above everything
    assert np.signbit(values[0, 4]) and not np.signbit(values[0, 2])


def test_topk_brute_force_python_sort():
    rng = np.random.default_rng(5)
    scores = rng.integers(-3, 4, size=(4, 50)).astype(np.float32)  # many ties
    values, ids = topk.exact_topk(scores, 20)
    for r in range(4):
        order = sorted(range(50), key=lambda j: (-scores[r, j], j))[:20]
        assert ids[r].tolist() == order


def test_digit_counts_pins():
    """Counts sum to the columns; equal a per-element loop over the float bits
    (struct, no numpy views); the suffix count reaches k in the bucket that
    holds exact_topk's k-th value."""
    import struct

    rng = np.random.default_rng(9)
    scores = (rng.standard_normal((5, 700)) * rng.choice([1e-30, 1.0, 1e30], (5, 700))).astype(np.float32)
    scores[0, ::7] = -np.inf
    scores[1, :300] = 0.0
    scores[1, 300:310] = -0.0
    scores[2, 5] = np.nan
    scores[3, 9] = np.inf
    counts = topk.digit_counts(scores)
    assert counts.shape == (5, 2048) and (counts.sum(axis=1) == 700).all()
    for r in range(2):
        loop = [0] * 2048
        for v in scores[r].tolist():
            (b,) = struct.unpack("<I", struct.pack("<f", v))
            key = (~b & 0xFFFFFFFF) if b >> 31 else (b | 0x80000000)
            loop[key >> 21] += 1
        assert counts[r].tolist() == loop
    for k in (1, 17, 350, 700):
        values, _ = topk.exact_topk(scores, k)
        for r in range(5):
            suffix = np.cumsum(counts[r][::-1])[::-1]  # keys at or above each bucket
            bucket = int(np.nonzero(suffix >= k)[0].max())
            kth = topk.radix_keys(values[r, k - 1:k])[0] >> 21
            assert bucket == kth
