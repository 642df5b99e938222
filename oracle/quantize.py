"""A1: per-row fp8-e4m3 quantisation with an fp32 scale (TEST INFRASTRUCTURE ONLY).

Restates the reference's device path, ``quantize_kernel`` in
``operators/deepseek_v32/indexer/quantization.py:34-60``, which its own tests
require to equal the eager formula ``reference_quantize_index``
(``quantization.py:12-21``) bit-for-bit on the GPU
(``indexer/tests/test_quantization.py:84-134``):

* ``amax = max(|x|)`` over the last axis, NaN-propagating, then
  ``max(amax, 1e-4)`` (NaN stays NaN);
* ``scale = amax * fl32(1/448)`` - the reference's GPU divide by a scalar
  multiplies by the fp32 reciprocal (``quantization.py:44-45``);
* UE8M0: ``scale`` is rounded up to a power of two,
  ``(bits + 0x7FFFFF) & 0x7F800000`` (``quantization.py:46-52``), equal to
  ``exp2(ceil(log2(scale)))`` on the bf16 amax domain;
* ``y = clamp(x / scale, -448, 448)`` (``x * (1/scale)`` for UE8M0, the same
  value because the scale is a power of two), cast to e4m3fn with RNE;
* NaN follows the reference GPU's canonical NaN: scale bits 0x7FFFFFFF and
  data code 0x7F.

The CPU eager reference divides ``amax / 448`` exactly instead; for the UE8M0
default both agree on every bf16 amax (pinned in the tests), for
``scale_fmt=None`` they can differ by one ulp of the scale and this oracle
follows the GPU path.

Pinned by ``tests/test_oracle_fp8_quantize.py``: all 65,536 bf16 encodings as the
row maximum against torch's ``exp2(ceil(log2(.)))`` formulation and float8
cast, the reference test's non-finite rows and e4m3 midpoints at six row
scales, and closed-form scale values.
"""

import numpy as np

from oracle import fp8

RECIPROCAL_448 = np.float32(1.0) / np.float32(448.0)
CANONICAL_NAN_BITS = np.uint32(0x7FFFFFFF)


def row_scales(x, scale_fmt="ue8m0"):
    """float32 ``[..., D]`` -> float32 ``[..., 1]`` scales (GPU semantics)."""
    if scale_fmt not in ("ue8m0", None):
        raise ValueError("Unsupported indexer quantization scale format")
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=-1, keepdims=True)  # numpy max propagates NaN
    amax = np.where(np.isnan(amax), amax, np.maximum(amax, np.float32(1e-4)))
    scale = (amax * RECIPROCAL_448).astype(np.float32)
    bits = np.ascontiguousarray(scale).view(np.uint32).copy()
    nan = bits > 0x7F800000
    if scale_fmt == "ue8m0":
        bits = np.where(nan, bits, (bits + np.uint32(0x7FFFFF)) & np.uint32(0x7F800000))
    bits = np.where(nan, CANONICAL_NAN_BITS, bits).astype(np.uint32)
    return bits.view(np.float32)


def quantize_index(x, scale_fmt="ue8m0"):
    """Return ``(codes uint8 [..., D], scales float32 [..., 1])``.

    ``x`` holds float32 values (bf16 inputs are exactly representable).
    """
    x = np.asarray(x, dtype=np.float32)
    scale = row_scales(x, scale_fmt)
    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        if scale_fmt == "ue8m0":
            y = x * (np.float32(1.0) / scale)
        else:
            y = x / scale
    y = y.astype(np.float32)
    nan = np.isnan(y)
    y = np.clip(y, np.float32(-448.0), np.float32(448.0))
    codes = fp8.encode(np.where(nan, np.float32(0.0), y))
    codes[nan] = 0x7F
    return codes, scale
