"""Indexer input producers: K LayerNorm, non-interleaved RoPE, fp8 quantise and
the head-weight fold (TEST INFRASTRUCTURE ONLY).

Restates the indexer half of the reference's projection step,
``models/deepseek_v32/projections.py``:

* ``_project_index_k`` (``:114-121``): ``F.layer_norm(index_wk(x).float(),
  (128,), weight, bias, eps).bfloat16()``;
* ``apply_rope_pair(index_q, index_k, angles, interleaved=False)``
  (``:236-238``; ``rotary.py:47-56,69-85``): the first ``2 * len(angles)``
  dims rotate, with the non-interleaved pairing (dim ``i`` with dim
  ``i + 32``), ``real = a*cos - b*sin``, ``imag = b*cos + a*sin`` in fp32 from
  the bf16 inputs, each product and sum rounded to fp32 (torch's elementwise
  CPU kernels), the result rounded to bf16; the other dims pass through;
* ``quantize_index`` of both (``:239-240``, the A1 rule in ``oracle.quantize``);
* the head weights (``:241-242``): ``((head_logits * 64**-0.5) * q_scale) *
  128**-0.5`` in fp32, ``head_logits = F.linear(x.float(), weights_proj)``.

The RoPE table is an input, as in the reference (``prepare_rotary_cache``,
``rotary.py:59-64``: ``cat(cos(angles), sin(angles))`` per row, and a row
index per token).

LayerNorm reduction order. torch's CPU kernel reduces with its own vectorised
Welford; the kernel on the GPU and this oracle fix one order instead, so that
they agree bit for bit: per row of 128, 16 partial sums of 8 consecutive
values (added left to right), then pairwise at distance 8, 4, 2, 1;
``mean = sum / 128``; ``var`` the same tree over ``(x - mean)**2``;
``rstd = 1 / sqrt(var + eps)`` (each rounded); ``y = ((x - mean) * rstd) * w
+ b`` with every operation rounded to fp32.

Pinned by ``tests/test_oracle_projections.py``: LayerNorm against
``torch.nn.functional.layer_norm`` (within 4 fp32 ulp of the output scale) and
against a float64 evaluation, zero-variance rows and bias/weight closed forms;
RoPE against complex multiplication ``(a + ib) e^{i theta}`` in float64, the
identity at angle 0, the quarter turn (exact swap with a sign) and norm
preservation, and with a planted interleaved pairing and a planted sign flip
that must fail; the producer end to end against torch's own CPU ops in the
reference's order (``F.layer_norm`` aside, which differs only in that order).
"""

import numpy as np

from oracle import fp8
from oracle import quantize as oquant

INDEX_DIM = 128
ROPE_DIM = 64
INV_SQRT_HEADS = np.float32(64 ** -0.5)
INV_SQRT_DIM = np.float32(128 ** -0.5)


def _tree_sum_128(x):
    """Sum over the last axis (128) in the fixed order described above."""
    x = np.asarray(x, dtype=np.float32)
    parts = x.reshape(*x.shape[:-1], 16, 8)
    s = parts[..., 0]
    for j in range(1, 8):
        s = (s + parts[..., j]).astype(np.float32)
    for half in (8, 4, 2, 1):
        s = (s[..., :half] + s[..., half:2 * half]).astype(np.float32)
    return s[..., 0]


def layer_norm_128(x, weight, bias, eps):
    """float32 ``[..., 128]`` -> float32, the fixed-order LayerNorm."""
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    b = np.asarray(bias, dtype=np.float32)
    inv_n = np.float32(1.0 / 128.0)
    mean = (_tree_sum_128(x) * inv_n).astype(np.float32)[..., None]
    d = (x - mean).astype(np.float32)
    var = (_tree_sum_128((d * d).astype(np.float32)) * inv_n).astype(np.float32)[..., None]
    rstd = (np.float32(1.0) / np.sqrt((var + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = ((d * rstd).astype(np.float32) * w).astype(np.float32)
    return (y + b).astype(np.float32)


def rope_non_interleaved(x, cos, sin):
    """Rotate the first ``2 * cos.shape[-1]`` dims of float32 ``x [T, ..., D]``.

    ``cos``/``sin``: float32 ``[T, half]``, broadcast over the middle axes.
    Returns float32 (the caller rounds to bf16).
    """
    x = np.asarray(x, dtype=np.float32)
    half = cos.shape[-1]
    shape = (cos.shape[0],) + (1,) * (x.ndim - 2) + (half,)
    c = np.asarray(cos, dtype=np.float32).reshape(shape)
    s = np.asarray(sin, dtype=np.float32).reshape(shape)
    a, b = x[..., :half], x[..., half:2 * half]
    real = ((a * c).astype(np.float32) - (b * s).astype(np.float32)).astype(np.float32)
    imag = ((b * c).astype(np.float32) + (a * s).astype(np.float32)).astype(np.float32)
    return np.concatenate([real, imag, x[..., 2 * half:]], axis=-1).astype(np.float32)


def round_bf16(x):
    """float32 -> the float32 value of its bf16 rounding (RNE)."""
    return fp8.bf16_bits_to_f32(fp8.f32_to_bf16_bits(x))


def index_k(k_proj_bits, weight, bias, eps, cos, sin):
    """Index K producer up to bf16: LayerNorm -> bf16 -> RoPE -> bf16.

    ``k_proj_bits``: uint16 bf16 bits ``[T, 128]`` (the ``index_wk`` output).
    Returns float32 values of bf16 ``[T, 128]``.
    """
    k = fp8.bf16_bits_to_f32(k_proj_bits)
    k = round_bf16(layer_norm_128(k, weight, bias, eps))
    return round_bf16(rope_non_interleaved(k, cos, sin))


def index_q(q_proj_bits, cos, sin):
    """Index Q producer up to bf16: RoPE -> bf16, ``[T, 64, 128]``."""
    q = fp8.bf16_bits_to_f32(q_proj_bits)
    return round_bf16(rope_non_interleaved(q, cos, sin))


def fold_weights(head_logits, q_scales):
    """``((head_logits * 64**-0.5) * q_scale) * 128**-0.5`` in fp32."""
    w = (np.asarray(head_logits, dtype=np.float32) * INV_SQRT_HEADS).astype(np.float32)
    w = (w * np.asarray(q_scales, dtype=np.float32)).astype(np.float32)
    return (w * INV_SQRT_DIM).astype(np.float32)


def index_producer(q_proj_bits, k_proj_bits, norm_weight, norm_bias, eps, cos_sin, rows,
                   head_logits):
    """The indexer half of ``project`` from the two GEMM outputs.

    ``cos_sin``: float32 ``[P, 64]`` (cos | sin of 32 angles per row),
    ``rows``: int ``[T]`` row of each token in it. Returns ``(q_codes
    [T,64,128], q_scales [T,64,1], k_codes [T,128], k_scales [T], weights
    [T,64])``.
    """
    table = np.asarray(cos_sin, dtype=np.float32)[np.asarray(rows)]
    cos, sin = table[:, :ROPE_DIM // 2], table[:, ROPE_DIM // 2:]
    q = index_q(q_proj_bits, cos, sin)
    k = index_k(k_proj_bits, norm_weight, norm_bias, eps, cos, sin)
    q_codes, q_scales = oquant.quantize_index(q)
    k_codes, k_scales = oquant.quantize_index(k)
    weights = fold_weights(head_logits, q_scales[..., 0])
    return q_codes, q_scales, k_codes, k_scales[:, 0], weights
