"""Pins of the oracle's fp8 codec and A1 quantiser (CPU only).

The checks use independent routes: torch's own float8 cast, torch's
``exp2(ceil(log2(.)))`` scale formulation, exact float64 products, and the
reference test's special rows (operators/deepseek_v32/indexer/tests/
test_quantization.py:84-134).
"""

import numpy as np
import pytest
import torch

from oracle import fp8, quantize


def all_bf16_values():
    return fp8.bf16_bits_to_f32(np.arange(65536, dtype=np.uint32).astype(np.uint16))


def test_encode_matches_torch_float8_cast_on_every_bf16_value():
    x = all_bf16_values()
    expected = torch.from_numpy(x.copy()).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(fp8.encode(x), expected)


def test_encode_matches_torch_on_random_fp32_and_midpoints():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(500_000).astype(np.float32) * np.float32(60),
        rng.standard_normal(100_000).astype(np.float32) * np.float32(1e-2),
        rng.uniform(-470, 470, 100_000).astype(np.float32),
    ])
    positive = fp8.decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mid = ((positive[:-1] + positive[1:]) / 2).astype(np.float32)
    x = np.concatenate([x, mid, -mid, np.nextafter(mid, 0), np.nextafter(mid, 1000)])
    expected = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(fp8.encode(x), expected)


def test_decode_matches_torch_on_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = fp8.decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    assert np.array_equal(np.isnan(ours), np.isnan(theirs))
    ok = ~np.isnan(ours)
    np.testing.assert_array_equal(ours[ok].view(np.uint32), theirs[ok].view(np.uint32))
    assert ours[0x7E] == 448 and ours[0x01] == 2.0**-9 and np.isnan(ours[0xFF])


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(200_000) * 10).astype(np.float32)
    x = np.concatenate([x, np.array([np.inf, -np.inf, 0.0, -0.0, 3.0e38, 1e-40], np.float32)])
    theirs = torch.from_numpy(x).bfloat16().view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(fp8.f32_to_bf16_bits(x), theirs)
    # NaN payloads are outside the contract; NaN stays NaN.
    nan = fp8.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(fp8.bf16_bits_to_f32(nan))[0]


def _torch_ue8m0(x):
    """torch's log2/ceil/exp2 formulation of the UE8M0 scale and the cast."""
    t = torch.from_numpy(x)
    amax = t.abs().amax(-1, keepdim=True).clamp_min(1e-4)
    scale = torch.exp2(torch.ceil(torch.log2(amax / 448.0)))
    codes = (t / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, scale.numpy()


def test_ue8m0_every_bf16_value_as_row_maximum_matches_log2_formulation():
    values = all_bf16_values()
    x = np.repeat(values[:, None], 128, axis=1)
    x[:, 1::2] *= -1
    codes, scales = quantize.quantize_index(x, "ue8m0")
    ref_codes, ref_scales = _torch_ue8m0(x)
    finite = np.isfinite(values)
    np.testing.assert_array_equal(scales[finite].view(np.uint32), ref_scales[finite].view(np.uint32))
    np.testing.assert_array_equal(codes[finite], ref_codes[finite])
    # Non-finite rows: NaN scale is the canonical 0x7FFFFFFF, inf stays inf.
    nan_rows = np.isnan(values)
    assert (scales[nan_rows].view(np.uint32) == 0x7FFFFFFF).all()
    assert (codes[nan_rows] == 0x7F).all()
    inf_rows = np.isinf(values)
    assert np.isinf(scales[inf_rows]).all()
    assert (codes[inf_rows] == 0x7F).all()  # +-inf * 0 is NaN


def test_none_format_scale_is_the_exactly_rounded_reciprocal_product():
    values = all_bf16_values()
    finite = np.isfinite(values) & (np.abs(values) >= 1e-4)
    amax = np.abs(values[finite]).astype(np.float32)
    x = np.repeat(amax[:, None], 128, axis=1)
    _, scales = quantize.quantize_index(x, None)
    recip = np.float64(np.float32(1.0) / np.float32(448.0))
    # float32 * float32 is exact in float64; one rounding to float32 follows.
    expected = (amax.astype(np.float64) * recip).astype(np.float32)
    np.testing.assert_array_equal(scales[:, 0].view(np.uint32), expected.view(np.uint32))


def test_known_scale_values():
    row = np.zeros((1, 128), np.float32)
    row[0, 0] = 448.0
    for fmt in ("ue8m0", None):
        codes, scales = quantize.quantize_index(row, fmt)
        assert scales[0, 0] == 1.0 and codes[0, 0] == 0x7E and (codes[0, 1:] == 0).all()
    row[0, 0] = 1.0
    codes, scales = quantize.quantize_index(row, "ue8m0")
    assert scales[0, 0] == 2.0**-8  # 1/448 rounded up to a power of two
    assert codes[0, 0] == fp8.encode(np.array([256.0], np.float32))[0]
    zero = np.zeros((1, 128), np.float32)
    codes, scales = quantize.quantize_index(zero, None)
    assert scales[0, 0] == np.float32(np.float32(1e-4) * (np.float32(1) / np.float32(448)))
    assert (codes == 0).all()


def test_reference_special_rows_match_log2_formulation():
    x = np.ones((8, 128), np.float32)
    x[0, 0] = np.inf
    x[1, 0] = -np.inf
    x[2, 0] = np.nan
    x[3] = np.nan
    x[4] = -np.inf
    x[5] = -0.0
    x[6, 0] = -np.nan
    x[7, 127] = np.nan
    codes, scales = quantize.quantize_index(x, "ue8m0")
    assert scales[5, 0] == 2.0**-22 and (codes[5] == 0x80).all()
    for r in (0, 1):
        assert np.isinf(scales[r, 0])
        assert codes[r, 0] == 0x7F and (codes[r, 1:] == 0).all()
    for r in (2, 3, 6, 7):
        assert scales[r, 0].view(np.uint32) == 0x7FFFFFFF and (codes[r] == 0x7F).all()
    assert np.isinf(scales[4, 0]) and (codes[4] == 0x7F).all()


def test_rounding_midpoints_at_six_scales_match_log2_formulation():
    positive = fp8.decode(np.arange(127, dtype=np.uint8)).astype(np.float64)
    middle = torch.from_numpy(((positive[:-1] + positive[1:]) / 2)).to(torch.bfloat16)
    samples = torch.stack((
        torch.nextafter(middle, torch.full_like(middle, -torch.inf)),
        middle,
        torch.nextafter(middle, torch.full_like(middle, torch.inf)),
    )).flatten()
    rows = []
    for factor in (2.0**-30, 2.0**-20, 2.0**-10, 1.0, 2.0**10, 2.0**60):
        for maximum in (448.0, 450.0, 510.0):
            x = torch.zeros(samples.numel(), 128, dtype=torch.bfloat16)
            x[:, 0] = maximum * factor
            x[:, 1] = samples * factor
            x[:, 2] = -samples * factor
            rows.append(x)
    x = torch.cat(rows).float().numpy()
    codes, scales = quantize.quantize_index(x, "ue8m0")
    ref_codes, ref_scales = _torch_ue8m0(x)
    np.testing.assert_array_equal(scales.view(np.uint32), ref_scales.view(np.uint32))
    np.testing.assert_array_equal(codes, ref_codes)


def test_unsupported_scale_format_is_rejected():
    with pytest.raises(ValueError, match="scale format"):
        quantize.quantize_index(np.ones((1, 128), np.float32), "packed")
