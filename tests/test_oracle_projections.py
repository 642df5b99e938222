"""Pins of the oracle's indexer input producers (CPU only).

``oracle.projections`` restates the indexer half of the reference's
projection step (``models/deepseek_v32/projections.py:114-121,236-244``,
``rotary.py:47-85``). Each pin uses a route that does not reuse the oracle's
arithmetic:

* LayerNorm against ``torch.nn.functional.layer_norm`` on CPU (the routine the
  reference calls; its reduction order differs, so within 4 fp32 ulp of the
  output scale) and against a float64 evaluation; a constant row gives the
  bias exactly; +-1 rows with unit weight and no eps give the input exactly;
* RoPE against complex multiplication ``(a + ib) e^{i theta}`` in float64
  (within 2 fp32 ulp), the identity at angle 0 (bit exact), the quarter turn
  (an exact swap with a sign change) and the pairing of dim ``i`` with
  ``i + 32`` on unit vectors;
* the producer end to end against torch CPU ops in the reference's order
  (``apply_rope`` and ``reference_quantize_index`` restated as torch calls,
  ``F.layer_norm``), with torch's LayerNorm the only step allowed to differ
  (counted: at most a few bf16 roundings in 10^5 may flip);
* the head weights against torch's ``(linear * 64**-0.5) * q_scale *
  128**-0.5`` bit for bit.

``test_pins_reject_planted_mistakes`` runs the checks on copies of the oracle
with a planted mistake (unbiased variance, interleaved pairing, a flipped
rotation sign, the weight fold without ``128**-0.5``, LayerNorm without the
bias) and requires each to fail.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import fp8
from oracle import projections as oproj


def _bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).bfloat16().view(
        torch.int16).numpy().view(np.uint16)


def _ln_inputs(rows, seed):
    rng = np.random.default_rng(seed)
    x = fp8.bf16_bits_to_f32(_bf16_bits(rng.standard_normal((rows, 128)) * 3 + 0.5))
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    return x, w, b


def _angles(tokens, seed):
    rng = np.random.default_rng(seed)
    positions = rng.integers(0, 70000, tokens).astype(np.float32)
    freq = (10000.0 ** (-np.arange(0, 64, 2, dtype=np.float32) / 64)).astype(np.float32)
    return (positions[:, None] * freq[None, :]).astype(np.float32)


# ----------------------------------------------------------------- the checks
def check_layer_norm_against_torch(impl):
    x, w, b = _ln_inputs(512, 1)
    ours = impl.layer_norm_128(x, w, b, 1e-6)
    ref = F.layer_norm(torch.from_numpy(x), (128,), torch.from_numpy(w), torch.from_numpy(b),
                       1e-6).numpy()
    scale = np.abs(ref).max(axis=-1, keepdims=True)
    assert (np.abs(ours - ref) <= 4 * np.finfo(np.float32).eps * scale).all()
    x64 = x.astype(np.float64)
    mean = x64.mean(-1, keepdims=True)
    var = ((x64 - mean) ** 2).mean(-1, keepdims=True)
    y64 = (x64 - mean) / np.sqrt(var + 1e-6) * w + b
    np.testing.assert_allclose(ours, y64, rtol=0, atol=1e-5)


def check_layer_norm_closed_forms(impl):
    _, w, b = _ln_inputs(1, 2)
    const = np.full((3, 128), 7.25, np.float32)
    np.testing.assert_array_equal(impl.layer_norm_128(const, w, b, 1e-6), np.broadcast_to(b, (3, 128)))
    signs = np.where(np.arange(128) % 3 == 0, 1.0, -1.0).astype(np.float32)
    signs = np.concatenate([signs[:64], -signs[:64]])  # mean exactly 0, variance exactly 1
    got = impl.layer_norm_128(signs[None], np.ones(128, np.float32), np.zeros(128, np.float32), 0.0)
    np.testing.assert_array_equal(got[0], signs)


def check_rope_against_complex(impl):
    rng = np.random.default_rng(3)
    angles = _angles(64, 4)
    x = fp8.bf16_bits_to_f32(_bf16_bits(rng.standard_normal((64, 5, 128))))
    got = impl.rope_non_interleaved(x, np.cos(angles), np.sin(angles))
    z = (x[..., :32].astype(np.float64) + 1j * x[..., 32:64]) * np.exp(
        1j * angles.astype(np.float64))[:, None, :]
    tol = 2 * np.finfo(np.float32).eps * (np.abs(x[..., :32]) + np.abs(x[..., 32:64]))
    assert (np.abs(got[..., :32] - z.real) <= tol + 1e-30).all()
    assert (np.abs(got[..., 32:64] - z.imag) <= tol + 1e-30).all()
    np.testing.assert_array_equal(got[..., 64:], x[..., 64:])


def check_rope_closed_forms(impl):
    rng = np.random.default_rng(5)
    x = fp8.bf16_bits_to_f32(_bf16_bits(rng.standard_normal((4, 2, 128))))
    zero = np.zeros((4, 32), np.float32)
    np.testing.assert_array_equal(impl.rope_non_interleaved(x, zero + 1, zero), x)
    # A quarter turn: cos 0, sin 1 -> (a, b) -> (-b, a) exactly.
    got = impl.rope_non_interleaved(x, zero, zero + 1)
    np.testing.assert_array_equal(got[..., :32], -x[..., 32:64])
    np.testing.assert_array_equal(got[..., 32:64], x[..., :32])
    # Pairing: a unit vector on dim 5 turns into dims 5 and 37 only.
    e = np.zeros((1, 128), np.float32)
    e[0, 5] = 1.0
    theta = np.float32(0.5)
    got = impl.rope_non_interleaved(e, np.full((1, 32), np.cos(theta), np.float32),
                                    np.full((1, 32), np.sin(theta), np.float32))
    expect = np.zeros((1, 128), np.float32)
    expect[0, 5], expect[0, 37] = np.cos(theta), np.sin(theta)
    np.testing.assert_array_equal(got, expect)


def _torch_quantize(x):
    """reference_quantize_index (quantization.py:12-21) as torch calls."""
    amax = x.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    scale = torch.exp2(torch.ceil(torch.log2(amax / 448.0)))
    return (x / scale).clamp(-448, 448).to(torch.float8_e4m3fn), scale


def _torch_rope(x, angles):
    """rotary.apply_rope(x, angles, interleaved=False) on the first 64 dims."""
    cos = angles.cos().reshape(angles.shape[0], *([1] * (x.ndim - 2)), -1)
    sin = angles.sin().reshape_as(cos)
    a, b = x[..., :64].float().chunk(2, -1)
    rot = torch.cat((a * cos - b * sin, b * cos + a * sin), -1).to(x.dtype)
    return torch.cat((rot, x[..., 64:]), -1)


def check_producer_against_torch(impl):
    rng = np.random.default_rng(6)
    tokens = 48
    q_bits = _bf16_bits(rng.standard_normal((tokens, 64, 128)))
    k_bits = _bf16_bits(rng.standard_normal((tokens, 128)) * 2)
    w = (1 + 0.1 * rng.standard_normal(128)).astype(np.float32)
    b = (0.1 * rng.standard_normal(128)).astype(np.float32)
    head = rng.standard_normal((tokens, 64)).astype(np.float32) * 4
    angles = torch.from_numpy(_angles(tokens, 7))
    cos_sin = torch.cat((angles.cos(), angles.sin()), -1).numpy()
    rows = np.arange(tokens)
    q8, qs, k8, ks, weights = impl.index_producer(q_bits, k_bits, w, b, 1e-6, cos_sin, rows, head)

    tq = torch.from_numpy(q_bits.view(np.int16)).view(torch.bfloat16)
    tk = torch.from_numpy(k_bits.view(np.int16)).view(torch.bfloat16)
    tk = F.layer_norm(tk.float(), (128,), torch.from_numpy(w), torch.from_numpy(b), 1e-6).bfloat16()
    rq8, rqs = _torch_quantize(_torch_rope(tq, angles).float())
    rk8, rks = _torch_quantize(_torch_rope(tk, angles).float())
    np.testing.assert_array_equal(q8, rq8.view(torch.uint8).numpy())
    np.testing.assert_array_equal(qs, rqs.numpy())
    # Index K: torch's LayerNorm reduces in another order; a bf16 rounding
    # (and then at most one e4m3 step) may flip on a rare value.
    diff = k8 != rk8.view(torch.uint8).numpy()
    assert diff.sum() <= 3, int(diff.sum())
    np.testing.assert_array_equal(ks, rks[:, 0].numpy())
    rw = torch.from_numpy(head) * 64 ** -0.5
    rw = rw * rqs[..., 0] * 128 ** -0.5
    np.testing.assert_array_equal(weights.view(np.uint32), rw.numpy().view(np.uint32))


CHECKS = [check_layer_norm_against_torch, check_layer_norm_closed_forms,
          check_rope_against_complex, check_rope_closed_forms, check_producer_against_torch]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_oracle_pins(check):
    check(oproj)


def test_rope_table_rows_index_tokens():
    """Token t uses row rows[t] of the table, not row t."""
    rng = np.random.default_rng(8)
    q_bits = _bf16_bits(rng.standard_normal((3, 64, 128)))
    k_bits = _bf16_bits(rng.standard_normal((3, 128)))
    table = np.concatenate([np.cos(_angles(10, 9)), np.sin(_angles(10, 9))], -1)
    head = np.ones((3, 64), np.float32)
    ones, zeros = np.ones(128, np.float32), np.zeros(128, np.float32)
    a = oproj.index_producer(q_bits, k_bits, ones, zeros, 1e-6, table, np.array([7, 2, 9]), head)
    b = oproj.index_producer(q_bits, k_bits, ones, zeros, 1e-6, table[[7, 2, 9]], np.arange(3),
                             head)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(x, y)


# ------------------------------------------------------------ planted mistakes
class _Mutant:
    def __init__(self, kind):
        self.kind = kind

    def layer_norm_128(self, x, weight, bias, eps):
        if self.kind == "unbiased_variance":
            x = np.asarray(x, np.float32)
            mean = x.mean(-1, keepdims=True, dtype=np.float32)
            var = ((x - mean) ** 2).sum(-1, keepdims=True, dtype=np.float32) / np.float32(127)
            return ((x - mean) / np.sqrt(var + np.float32(eps)) * weight + bias).astype(np.float32)
        if self.kind == "no_bias":
            return oproj.layer_norm_128(x, weight, np.zeros_like(bias), eps)
        return oproj.layer_norm_128(x, weight, bias, eps)

    def rope_non_interleaved(self, x, cos, sin):
        if self.kind == "interleaved":
            x = np.asarray(x, np.float32)
            shape = (cos.shape[0],) + (1,) * (x.ndim - 2) + (32,)
            c, s = cos.reshape(shape).astype(np.float32), sin.reshape(shape).astype(np.float32)
            a, b = x[..., 0:64:2], x[..., 1:64:2]
            out = np.stack([a * c - b * s, b * c + a * s], -1).reshape(*x.shape[:-1], 64)
            return np.concatenate([out, x[..., 64:]], -1).astype(np.float32)
        if self.kind == "flipped_sign":
            return oproj.rope_non_interleaved(x, cos, -np.asarray(sin))
        return oproj.rope_non_interleaved(x, cos, sin)

    def index_producer(self, q_bits, k_bits, w, b, eps, cos_sin, rows, head):
        table = np.asarray(cos_sin, np.float32)[rows]
        cos, sin = table[:, :32], table[:, 32:]
        q = oproj.round_bf16(self.rope_non_interleaved(fp8.bf16_bits_to_f32(q_bits), cos, sin))
        k = oproj.round_bf16(self.layer_norm_128(fp8.bf16_bits_to_f32(k_bits), w, b, eps))
        k = oproj.round_bf16(self.rope_non_interleaved(k, cos, sin))
        from oracle import quantize as oquant

        q8, qs = oquant.quantize_index(q)
        k8, ks = oquant.quantize_index(k)
        weights = oproj.fold_weights(head, qs[..., 0])
        if self.kind == "fold_without_dim_scale":
            weights = (weights / oproj.INV_SQRT_DIM).astype(np.float32)
        return q8, qs, k8, ks[:, 0], weights


@pytest.mark.parametrize("kind", ["unbiased_variance", "no_bias", "interleaved", "flipped_sign",
                                  "fold_without_dim_scale"])
def test_pins_reject_planted_mistakes(kind):
    mutant = _Mutant(kind)
    failures = 0
    for check in CHECKS:
        try:
            with np.errstate(all="ignore"):
                check(mutant)
        except AssertionError:
            failures += 1
    assert failures > 0, f"no pin detects the planted mistake {kind!r}"


def test_rotary_frequencies_closed_forms():
    """YaRN frequencies (rotary.py:26-44): unchanged below the low
    correction dim, divided by the factor above the high one."""
    from cxldsagr_amd.projections import rotary_frequencies

    plain = rotary_frequencies(64, 10000.0, 4096, 4096, 32.0, 1.0, 40.0).double().numpy()
    np.testing.assert_allclose(plain, 10000.0 ** (-np.arange(0, 64, 2) / 64), rtol=1e-6)
    yarn = rotary_frequencies(64, 10000.0, 163840, 4096, 32.0, 1.0, 40.0).double().numpy()

    def correction(rotations):
        return 64 * math.log(4096 / (rotations * 2 * math.pi)) / (2 * math.log(10000.0))

    low, high = math.floor(correction(32.0)), math.ceil(correction(1.0))
    assert (low, high) == (10, 23)
    np.testing.assert_allclose(yarn[:low + 1], plain[:low + 1], rtol=1e-6)
    np.testing.assert_allclose(yarn[high:], plain[high:] / 40.0, rtol=1e-6)
    mid = np.arange(low + 1, high)
    ramp = (mid - low) / (high - low)
    np.testing.assert_allclose(yarn[mid], plain[mid] * (1 - ramp) + plain[mid] / 40 * ramp, rtol=1e-5)
