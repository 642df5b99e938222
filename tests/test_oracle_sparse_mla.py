"""Pins of the oracle's sparse MLA (CPU only).

Three independent routes, none of which restates the oracle's vectorised
formula:

* the reference's own known answers, applied to the oracle:
  duplicates / padding -> 4, 0, 2 and RoPE dimensions that only steer the
  scores -> 0.75
  (operators/deepseek_v32/attention/reference/tests/test_deepseek_reference_mla.py:45-65),
  +-100 x 100 logits around empty tiles -> exactly 2
  (attention/device_only/tests/test_deepseek_mla.py:110-121), int64 ids that
  would wrap into valid rows when narrowed (:83-94), empty inputs -> zeros
  (:145-153);
* a float64 scalar-loop brute force on small random shapes with duplicates,
  -1 and out-of-range ids, int32 and int64 ids;
* closed forms: one valid key -> its value row exactly; equal scores -> the
  plain mean of the selected value rows.

``test_pins_reject_planted_mistakes`` runs the same checks against copies of
the oracle with a planted mistake (no max subtraction, padding ids kept, the
RoPE dims dropped from the scores, the value slice taken from the RoPE end,
the softmax taken over heads) and requires each copy to fail at least one of
them.
"""

import math

import numpy as np
import pytest

from oracle import fp8
from oracle import sparse_mla as omla


def _f32(out_bits):
    return fp8.bf16_bits_to_f32(out_bits)


# ----------------------------------------------------------------- the checks
# Each takes a sparse-MLA function with the oracle's signature and raises
# AssertionError when it disagrees with the pinned answer.

def check_duplicates_and_padding(fn):
    q = np.zeros((3, 2, 24), np.float32)
    kv = np.zeros((3, 24), np.float32)
    kv[0] = np.nan
    kv[1, :16] = 2
    kv[2, :16] = 5
    ids = np.array([[1, 2, 2, -1], [-1, -1, 10, -1], [1, -1, -1, -1]])
    with np.errstate(all="ignore"):
        _, out = fn(q, kv, ids, 1.0, 16)
    np.testing.assert_allclose(out[0], np.full((2, 16), 4.0), rtol=1e-6)
    np.testing.assert_array_equal(out[1], np.zeros((2, 16)))
    np.testing.assert_allclose(out[2], np.full((2, 16), 2.0), rtol=1e-6)


def check_rope_steers_scores_only(fn):
    q = np.zeros((1, 1, 24), np.float32)
    q[..., 23] = 1
    kv = np.zeros((2, 24), np.float32)
    kv[1, :16] = 1
    kv[1, 23] = math.log(3)
    _, out = fn(q, kv, np.array([[0, 1]]), 1.0, 16)
    np.testing.assert_allclose(out, np.full((1, 1, 16), 0.75), rtol=1e-6)


def check_large_logits_exact(fn):
    q = np.zeros((1, 64, 576), np.float32)
    q[..., 575] = 100
    kv = np.zeros((3, 576), np.float32)
    kv[0] = np.nan
    kv[1, :512], kv[1, 575] = 2, 100
    kv[2, :512], kv[2, 575] = 5, -100
    ids = np.full((1, 193), -1, np.int64)
    ids[0, 65:67] = [1, 2]
    with np.errstate(all="ignore"):
        bits, out = fn(q, kv, ids, 1.0, 512)
    assert np.array_equal(_f32(bits), np.full((1, 64, 512), 2.0, np.float32))


def check_int64_ids_do_not_wrap(fn):
    q = np.zeros((2, 64, 576), np.float32)
    kv = np.full((4, 576), 7, np.float32)
    kv[0] = np.nan
    kv[1, :512] = 2
    ids = np.full((2, 129), 2**32 + 1, np.int64)
    ids[0, 1] = -(2**32) + 1
    ids[1, 0] = 1
    with np.errstate(all="ignore"):
        bits, _ = fn(q, kv, ids, 1.0, 512)
    out = _f32(bits)
    assert np.array_equal(out[0], np.zeros_like(out[0]))
    assert np.array_equal(out[1], np.full_like(out[1], 2.0))


def check_brute_force(fn, seed):
    rng = np.random.default_rng(seed)
    rows, heads, dim, value_dim, n = 3, 2, 24, 16, 9
    q = rng.standard_normal((rows, heads, dim)).astype(np.float32)
    kv = rng.standard_normal((n, dim)).astype(np.float32)
    ids = rng.integers(-2, n + 3, (rows, 7))
    ids[0, :3] = 4                      # duplicates
    ids[1] = -1                         # an all-padding row
    ids[2, 0], ids[2, 1] = n, 2**33     # out of range (int64)
    scale = 0.37
    _, got = fn(q, kv, ids, scale, value_dim)
    expected = omla.sparse_mla_brute_force(q, kv, ids, scale, value_dim)
    np.testing.assert_allclose(got, expected, rtol=2e-6, atol=2e-6)
    assert not got[1].any()


def check_closed_forms(fn):
    rng = np.random.default_rng(11)
    q = rng.standard_normal((2, 3, 24)).astype(np.float32)
    kv = rng.standard_normal((6, 24)).astype(np.float32)
    # One valid key (the rest padding): the output is that key's value row.
    ids = np.array([[5, -1, -1], [-1, 2, 17]])
    _, out = fn(q, kv, ids, 0.5, 16)
    np.testing.assert_allclose(out[0], np.broadcast_to(kv[5, :16], (3, 16)), rtol=1e-6)
    np.testing.assert_allclose(out[1], np.broadcast_to(kv[2, :16], (3, 16)), rtol=1e-6)
    # Zero queries give equal scores: the plain mean of the selected values.
    zero = np.zeros_like(q)
    ids = np.array([[0, 1, 3], [2, 2, 4]])
    _, out = fn(zero, kv, ids, 0.5, 16)
    np.testing.assert_allclose(out[0], np.broadcast_to(kv[[0, 1, 3], :16].mean(0), (3, 16)),
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out[1], np.broadcast_to(kv[[2, 2, 4], :16].mean(0), (3, 16)),
                               rtol=1e-5, atol=1e-6)


def check_empty(fn):
    for queries, tokens, selected in ((0, 5, 3), (2, 0, 3), (2, 5, 0)):
        q = np.zeros((queries, 4, 24), np.float32)
        kv = np.zeros((tokens, 24), np.float32)
        ids = np.full((queries, selected), -1, np.int64)
        bits, out = fn(q, kv, ids, 0.2, 16)
        assert out.shape == (queries, 4, 16) and not out.any() and not bits.any()


CHECKS = [
    check_duplicates_and_padding,
    check_rope_steers_scores_only,
    check_large_logits_exact,
    check_int64_ids_do_not_wrap,
    lambda fn: check_brute_force(fn, 0),
    lambda fn: check_brute_force(fn, 1),
    check_closed_forms,
    check_empty,
]


@pytest.mark.parametrize("check", range(len(CHECKS)))
def test_oracle_passes_pin(check):
    CHECKS[check](omla.sparse_mla)


def test_brute_force_on_random_shapes():
    for seed in range(2, 6):
        check_brute_force(omla.sparse_mla, seed)


def test_brute_force_reproduces_the_reference_known_answer():
    """The brute force itself agrees with the reference's 4 / 0 / 2 answer."""
    q = np.zeros((3, 2, 24))
    kv = np.zeros((3, 24))
    kv[1, :16] = 2
    kv[2, :16] = 5
    ids = np.array([[1, 2, 2, -1], [-1, -1, 10, -1], [1, -1, -1, -1]])
    out = omla.sparse_mla_brute_force(q, kv, ids, 1.0, 16)
    np.testing.assert_allclose(out[0], 4.0)
    np.testing.assert_allclose(out[1], 0.0)
    np.testing.assert_allclose(out[2], 2.0)


# ------------------------------------------------------------ planted mistakes
def _mutant(kind):
    def fn(q, kv, indices, scale, value_dim=512):
        q = np.asarray(q, dtype=np.float32)
        kv = np.asarray(kv, dtype=np.float32)
        indices = np.asarray(indices).astype(np.int64)
        rows, heads, _ = q.shape
        out = np.zeros((rows, heads, value_dim), dtype=np.float32)
        for r in range(rows):
            sel = indices[r]
            if kind != "keeps_padding":
                sel = sel[(sel >= 0) & (sel < kv.shape[0])]
            else:
                sel = sel[sel < kv.shape[0]]
            if not sel.size:
                continue
            records = kv[sel]
            if kind == "no_rope_in_scores":
                logits = (q[r, :, :value_dim] @ records[:, :value_dim].T) * np.float32(scale)
            else:
                logits = (q[r] @ records.T) * np.float32(scale)
            if kind == "softmax_over_heads":
                logits = logits - logits.max(axis=0, keepdims=True)
                p = np.exp(logits)
                p /= p.sum(axis=0, keepdims=True)
            else:
                if kind != "no_max_subtraction":
                    logits = logits - logits.max(axis=-1, keepdims=True)
                p = np.exp(logits)
                p /= p.sum(axis=-1, keepdims=True)
            values = records[:, -value_dim:] if kind == "value_from_end" else records[:, :value_dim]
            out[r] = p @ values
        return fp8.f32_to_bf16_bits(out), out

    return fn


@pytest.mark.parametrize("kind", ["no_max_subtraction", "keeps_padding", "no_rope_in_scores",
                                  "value_from_end", "softmax_over_heads"])
def test_pins_reject_planted_mistakes(kind):
    fn = _mutant(kind)
    failures = 0
    for check in CHECKS:
        try:
            with np.errstate(all="ignore"):
                check(fn)
        except (AssertionError, IndexError, ValueError, FloatingPointError):
            failures += 1
    assert failures > 0, f"no pin detects the planted mistake {kind!r}"
