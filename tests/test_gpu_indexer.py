"""GPU parity of the indexer kernels (A1 quantise, A4 logits, A6 top-k) with the oracle.

Cases follow the reference's own tests:
operators/deepseek_v32/indexer/tests/test_quantization.py,
test_echo_indexer.py and test_selection.py.
"""

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import logits as ologits
from oracle import quantize as oquant
from oracle import topk as otopk

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int32).numpy()


def _quant_check(x, scale_fmt):
    from cxldsagr_amd.indexer import quantize_index

    data, scales = quantize_index(x, scale_fmt)
    assert data.dtype == torch.float8_e4m3fn and scales.dtype == torch.float32
    assert data.is_contiguous() and scales.is_contiguous()
    assert data.shape == x.shape and scales.shape == (*x.shape[:-1], 1)
    ref_codes, ref_scales = oquant.quantize_index(x.detach().float().cpu().numpy(), scale_fmt)
    np.testing.assert_array_equal(data.view(torch.uint8).cpu().numpy(), ref_codes)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ref_scales.view(np.uint32))


# ----------------------------------------------------------------------------- A1


@pytest.mark.parametrize("scale_fmt", ["ue8m0", None])
@pytest.mark.parametrize("tokens,heads", [(0, 64), (1, 1), (17, 64), (128, 1), (1024, 64)])
def test_quantize_random_and_zero_rows(gpu, scale_fmt, tokens, heads):
    generator = torch.Generator(device="cuda").manual_seed(222)
    shape = (tokens, heads, 128) if heads != 1 else (tokens, 128)
    x = torch.randn(shape, generator=generator, device=gpu, dtype=torch.bfloat16)
    if tokens:
        x[0] = 0
    _quant_check(x, scale_fmt)


@pytest.mark.parametrize("scale_fmt", ["ue8m0", None])
def test_quantize_every_bf16_value_as_row_maximum(gpu, scale_fmt):
    values = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    x = values[:, None].expand(-1, 128).contiguous().to(gpu)
    x[:, 1::2] *= -1
    _quant_check(x, scale_fmt)


@pytest.mark.parametrize("scale_fmt", ["ue8m0", None])
def test_quantize_nonfinite_values_poison_the_row(gpu, scale_fmt):
    x = torch.ones(8, 128, dtype=torch.bfloat16, device=gpu)
    x[0, 0] = torch.inf
    x[1, 0] = -torch.inf
    x[2, 0] = torch.nan
    x[3].fill_(torch.nan)
    x[4].fill_(-torch.inf)
    x[5].fill_(-0.0)
    x[6, 0] = -torch.nan
    x[7, 127] = torch.nan
    _quant_check(x, scale_fmt)


@pytest.mark.parametrize("scale_fmt", ["ue8m0", None])
def test_quantize_fp8_rounding_boundaries_and_tiny_values(gpu, scale_fmt):
    positive = torch.arange(127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    middle = ((positive[:-1] + positive[1:]) / 2).to(torch.bfloat16)
    samples = torch.stack(
        (
            torch.nextafter(middle, torch.full_like(middle, -torch.inf)),
            middle,
            torch.nextafter(middle, torch.full_like(middle, torch.inf)),
        )
    ).flatten()
    rows = []
    for factor in (2.0**-30, 2.0**-20, 2.0**-10, 1.0, 2.0**10, 2.0**60):
        for maximum in (448.0, 450.0, 510.0):
            x = torch.zeros(samples.numel(), 128, dtype=torch.bfloat16)
            x[:, 0] = maximum * factor
            x[:, 1] = samples * factor
            x[:, 2] = -samples * factor
            rows.append(x)
    _quant_check(torch.cat(rows).to(gpu), scale_fmt)


@pytest.mark.parametrize("scale_fmt", ["ue8m0", None])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_quantize_layouts_and_dtypes(gpu, scale_fmt, dtype):
    source = torch.randn(17, 4, 256, device=gpu, dtype=dtype)
    for x in (source[..., ::2], source.transpose(0, 1), source[:, :, :127], source[0, 0],
              source[:, 0, :128]):
        _quant_check(x, scale_fmt)


# ----------------------------------------------------------------------------- A4


def _logit_inputs(rows, columns, device, seed=521):
    torch.manual_seed(seed)
    q = torch.randn(rows, 64, 128).to(torch.float8_e4m3fn).to(device)
    k = torch.randn(columns, 128).to(torch.float8_e4m3fn).to(device)
    weights = (torch.randn(rows, 64) / 64).to(device)
    scales = (torch.rand(columns) + 0.5).to(device)
    return q, k, weights, scales


def _oracle_logits(q, k, weights, scales, query_start, **kw):
    return ologits.logits(
        q.view(torch.uint8).cpu().numpy(),
        k.view(torch.uint8).cpu().numpy(),
        weights.cpu().numpy(),
        scales.cpu().numpy(),
        query_start,
        **kw,
    )


def _assert_logits_close(actual, expected):
    actual = actual.cpu().numpy()
    finite = np.isfinite(expected)
    # -inf exactly where the oracle masks, finite elsewhere.
    np.testing.assert_array_equal(np.isneginf(actual), ~finite)
    # Tolerance of the reference's own test (test_echo_indexer.py:109):
    # fp8 MFMA accumulation is not an IEEE fp32 dot product.
    np.testing.assert_allclose(actual[finite], expected[finite], atol=2e-3, rtol=1e-3)


@pytest.mark.parametrize(
    "rows,columns,query_start",
    [(1, 17, 16), (5, 4099, 4094), (302, 4096, 3794), (5, 23, 2), (17, 4099, 0), (1, 1, 0),
     (33, 65, 3), (128, 4224, 4096)],
)
def test_logits_match_fp32_oracle(gpu, rows, columns, query_start):
    from cxldsagr_amd.indexer import logits

    q, k, w, s = _logit_inputs(rows, columns, gpu)
    result = logits(q, k, w, s, query_start)
    assert result.shape == (rows, columns)
    padded = logits(q, k, w, s, query_start, _pad_to_stride=True)
    assert padded.shape == (rows, (columns + 255) // 256 * 256) and padded.is_contiguous()
    assert result.stride() == padded.stride()
    expected = _oracle_logits(q, k, w, s, query_start, pad_to_stride=True)
    _assert_logits_close(padded, expected)
    assert torch.equal(padded[:, :columns].view(torch.int32), result.view(torch.int32))


def test_logits_config1_shape(gpu):
    """Config 1 shape: 128 queries over 65536 history (+128 causal tail)."""
    from cxldsagr_amd.indexer import logits

    rows, columns = 128, 65664
    q, k, w, s = _logit_inputs(rows, columns, gpu, seed=947)
    result = logits(q, k, w, s, columns - rows, _pad_to_stride=True)
    expected = _oracle_logits(q, k, w, s, columns - rows, pad_to_stride=True)
    _assert_logits_close(result, expected)


def test_logits_bounds_zero_weights_and_repeat_bit_exact(gpu):
    from cxldsagr_amd.indexer import logits

    rows, columns, start = 40, 3000, 2960
    q, k, w, s = _logit_inputs(rows, columns, gpu)
    ends = torch.arange(start + 1, start + rows + 1, dtype=torch.int32, device=gpu)
    starts = torch.zeros(rows, dtype=torch.int32, device=gpu)
    a = logits(q, k, w, s, start)
    b = logits(q, k, w, s, start, _bounds=(starts, ends))
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))
    for _ in range(8):
        c = logits(q, k, w, s, start)
        assert torch.equal(a.view(torch.int32), c.view(torch.int32))
    zero = logits(q, k, torch.zeros_like(w), s, start)
    visible = torch.arange(columns, device=gpu)[None] < ends[:, None]
    assert zero[visible].eq(0).all() and torch.isneginf(zero[~visible]).all()


def _relu_rewrite_bound(q, k, w, s):
    """Bound on |kernel - exact| per (query, key) for the kernel's head sum.

    The kernel forms relu(s_h) w_h as (|s_h| + s_h) w_h / 2: the |s_h| half by
    fp32 FMAs, the linear half as k . q' with q' = sum_h (w_h / 2) q_h carried
    in four e4m3 digits (each digit the residual of the ones before to half an
    e4m3 ulp: |q'_d - digits_d| <= 2^-16 max|q'|). With M = sum_h |w_h| sum_d
    |q_hd k_d| and B = ||k||_1 max_d sum_h |w_h q_hd|, the fp32 dot products
    and FMA chains add at most 2^-17 M + 2^-18 M + 2^-19 M and the digits and
    the linear MFMA at most 2^-17 B + 2^-17 B, so |error| <= 2^-15 (M + B)
    times the key scale, with room to spare. Keys whose 64 head products are
    all negative are exactly 0 in the reference; here they are within it.
    """
    qd = q.float().double().cpu()
    kd = k.float().double().cpu()
    wd = w.double().cpu()
    sd = s.double().cpu()
    m = torch.einsum("qh,qhd,jd->qj", wd.abs(), qd.abs(), kd.abs())
    b = kd.abs().sum(1)[None, :] * (wd.abs()[:, :, None] * qd.abs()).sum(1).amax(1)[:, None]
    exact = torch.einsum("qh,qhj->qj", wd, torch.einsum("qhd,jd->qhj", qd, kd).clamp_min(0))
    return exact * sd[None, :], 2.0**-15 * (m + b) * sd[None, :]


def test_logits_relu_rewrite_bound_and_all_negative_keys(gpu):
    """Keys whose 64 head dot products are all negative give exactly 0 in the
    reference; the kernel's (|s| + s) / 2 rewrite leaves a residue that must
    stay inside the stated bound, as must every other key's error."""
    from cxldsagr_amd.indexer import logits

    torch.manual_seed(77)
    rows, columns = 12, 1536
    q = torch.randn(rows, 64, 128).abs().to(torch.float8_e4m3fn)
    k = torch.randn(columns, 128).to(torch.float8_e4m3fn)
    negative = torch.zeros(columns, dtype=torch.bool)
    negative[::2] = True
    k[negative] = (-(torch.randn(int(negative.sum()), 128).abs() + 0.05)).to(torch.float8_e4m3fn)
    w = torch.randn(rows, 64) * torch.logspace(-2, 1, rows)[:, None]  # both signs, wide range
    s = torch.rand(columns) + 0.5
    start = columns - rows
    out = logits(q.to(gpu), k.to(gpu), w.to(gpu), s.to(gpu), start).cpu().double()
    exact, bound = _relu_rewrite_bound(q, k, w, s)
    visible = torch.arange(columns)[None, :] < (start + 1 + torch.arange(rows))[:, None]
    assert torch.isneginf(out[~visible]).all()
    err = (out - exact).abs()[visible]
    assert (err <= bound[visible]).all(), float((err / bound[visible]).max())
    zero_keys = visible & negative[None, :]
    assert exact[zero_keys].eq(0).all()
    residue = out[zero_keys].abs()
    assert (residue <= bound[zero_keys]).all()
    # The bound is tight enough to matter: far below the size of the logits.
    assert float(bound[visible].max()) < 1e-2 * float(exact[visible].abs().max())
    print(f"all-negative keys: max |residue| {float(residue.max()):.3e}, "
          f"max residue / bound {float((residue / bound[zero_keys]).max()):.3f}; "
          f"all keys: max err / bound {float((err / bound[visible]).max()):.3f}")


def test_logits_rejects_invalid_inputs(gpu):
    from cxldsagr_amd.indexer import logits

    q, k, w, s = _logit_inputs(4, 64, gpu)
    with pytest.raises(ValueError, match="query_start"):
        logits(q, k, w, s, 61)
    with pytest.raises(ValueError, match="weights"):
        logits(q, k, w.double(), s, 0)
    with pytest.raises(NotImplementedError, match="prefetch"):
        logits(q, k, w, s, 0, prefetch={})


# ----------------------------------------------------------------------------- A6


def _topk_check(scores, k):
    from cxldsagr_amd.indexer import exact_topk

    values, indices = exact_topk(scores, k)
    ref_values, ref_ids = otopk.exact_topk(scores.cpu().numpy(), k)
    assert values.dtype == torch.float32 and indices.dtype == torch.int32
    np.testing.assert_array_equal(values.cpu().numpy().view(np.uint32), ref_values.view(np.uint32))
    np.testing.assert_array_equal(indices.cpu().numpy(), ref_ids)
    return values, indices


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_quantize_with_folded_weights(gpu, dtype):
    """The fused weight fold equals quantize_index followed by the fp32 product."""
    from cxldsagr_amd.indexer import quantize_index, quantize_index_folded

    generator = torch.Generator(device="cuda").manual_seed(31)
    x = (torch.randn(37, 64, 128, device=gpu, generator=generator) * 3).to(dtype)
    x[3, 5] = float("nan")
    weights = torch.randn(37, 64, device=gpu, generator=generator)
    data, scales = quantize_index(x)
    fdata, fscales, folded = quantize_index_folded(x, weights)
    assert torch.equal(fdata.view(torch.uint8), data.view(torch.uint8))
    assert torch.equal(fscales.view(torch.int32), scales.view(torch.int32))
    expected = weights * scales[..., 0]
    assert torch.equal(folded.view(torch.int32), expected.view(torch.int32))
    with pytest.raises(ValueError, match="weights must be FP32"):
        quantize_index_folded(x, weights[:, :32])


@pytest.mark.parametrize(
    "rows,columns,k",
    [(1, 1, 1), (3, 17, 2048), (5, 257, 32), (32, 4099, 1024), (64, 1024, 2048),
     (16, 65536, 1), (24, 66560, 2048), (4, 69633, 2048), (8, 131584, 2048)],
)
def test_topk_bit_exact_with_causal_masks(gpu, rows, columns, k):
    generator = torch.Generator(device="cuda").manual_seed(191)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    start = max(0, columns - rows)
    ends = (start + torch.arange(rows, device=gpu) + 1).clamp_max(columns)
    scores.masked_fill_(torch.arange(columns, device=gpu)[None] >= ends[:, None], -torch.inf)
    values, indices = _topk_check(scores, k)
    reference = scores.topk(min(k, columns), dim=-1)
    torch.testing.assert_close(values, reference.values, atol=0, rtol=0)


@pytest.mark.parametrize("rows,columns,k", [(3, 8191, 2048), (5, 8193, 2048), (7, 40001, 777),
                                             (2, 139264, 2048), (9, 65664, 2048)])
def test_topk_two_part_rows_equal_one_part_kernel(gpu, rows, columns, k):
    """The split entry (two work-groups per row, merged through the workspace)
    returns exactly what the one-work-group entry returns, call after call."""
    from cxldsagr_amd import _native
    from cxldsagr_amd.indexer import exact_topk

    generator = torch.Generator(device="cuda").manual_seed(columns)
    scores = torch.randn(rows, columns, device=gpu, generator=generator)
    scores[0, ::3] = 0.5  # ties across the two halves
    count = min(k, columns)
    values = torch.empty(rows, count, device=gpu)
    indices = torch.empty(rows, count, device=gpu, dtype=torch.int32)
    with torch.cuda.device(gpu):
        _native.call("dsa_topk_radix", _native.ptr(scores), rows, columns, scores.stride(0), k,
                     _native.ptr(values), _native.ptr(indices), count, _native.stream_of(gpu))
    for _ in range(3):
        split_values, split_indices = exact_topk(scores, k)
        assert torch.equal(split_values.view(torch.int32), values.view(torch.int32))
        assert torch.equal(split_indices, indices)


def test_topk_split_rejects_a_short_workspace(gpu):
    from cxldsagr_amd import _native

    scores = torch.randn(4, 9000, device=gpu)
    values = torch.empty(4, 2048, device=gpu)
    indices = torch.empty(4, 2048, device=gpu, dtype=torch.int32)
    workspace = torch.zeros(1024, dtype=torch.uint8, device=gpu)
    with pytest.raises(ValueError, match="workspace too small"):
        _native.call("dsa_topk_radix_split", _native.ptr(scores), 4, 9000, 9000, 2048,
                     _native.ptr(values), _native.ptr(indices), 2048, _native.ptr(workspace),
                     workspace.numel(), _native.stream_of(gpu))


def test_topk_misaligned_rows_stream_from_memory(gpu):
    """Rows that do not start on a 16-byte boundary take the scalar streaming path."""
    generator = torch.Generator(device="cuda").manual_seed(7)
    base = torch.randn(6, 70004, device=gpu, generator=generator)
    for offset, width in ((1, 70001), (3, 4099)):
        scores = base[:, offset:offset + width]
        assert scores.data_ptr() % 16
        _topk_check(scores, 2048)


def test_topk_every_k_small_ties(gpu):
    scores = -torch.arange(2049, device=gpu, dtype=torch.float32).remainder(19)
    scores = scores.expand(3, -1).clone()
    scores[1].fill_(-torch.inf)
    scores[2, 31:] = -torch.inf
    for k in (1, 2, 3, 18, 19, 20, 31, 32, 100, 107, 108, 109, 1000, 2047, 2048):
        _topk_check(scores, k)


def test_topk_large_tie_overflow_and_invalid_rows(gpu):
    from cxldsagr_amd.indexer import exact_topk

    scores = torch.zeros(3, 66560, device=gpu)
    scores[1].fill_(-torch.inf)
    scores[2, 7:] = -torch.inf
    expected = torch.arange(2048, device=gpu, dtype=torch.int32).expand(3, -1).clone()
    expected[1].fill_(-1)
    expected[2, 7:] = -1
    for _ in range(4):
        values, indices = exact_topk(scores, 2048)
        assert torch.equal(indices, expected)
        assert values[0].eq(0).all() and values[1].isneginf().all()


def test_topk_signed_zero_extremes_and_strides(gpu):
    base = torch.tensor(
        [torch.finfo(torch.float32).min, -1e30, -1e-30, -0.0, 0.0, 1e-30, 1e30,
         torch.finfo(torch.float32).max, -torch.inf],
        device=gpu,
    )
    scores = base.expand(5, -1).clone().T.contiguous().T
    assert not scores.is_contiguous()
    before = scores.clone()
    for k in (1, 2, 4, 5, 8, 9):
        _topk_check(scores, k)
    assert torch.equal(scores, before)
    rows = torch.tensor([[-0.0, 0.0, -0.0, 0.0, 1.0, -1.0]], device=gpu)
    values, indices = _topk_check(rows, 6)
    assert indices.tolist() == [[4, 1, 3, 0, 2, 5]]


def test_topk_padded_logits_view(gpu):
    """Top-k over the padded logits storage equals top-k over the logical view."""
    from cxldsagr_amd.indexer import exact_topk, logits

    rows, columns = 5, 4099
    q, k, w, s = _logit_inputs(rows, columns, gpu)
    original = logits(q, k, w, s, columns - rows)
    padded = logits(q, k, w, s, columns - rows, _pad_to_stride=True)
    for a, b in zip(exact_topk(padded, 2048), exact_topk(original, 2048)):
        assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_topk_empty_and_rejections(gpu):
    from cxldsagr_amd.indexer import exact_topk

    values, indices = exact_topk(torch.empty(0, 7, device=gpu), 2048)
    assert values.shape == indices.shape == (0, 7) and indices.dtype == torch.int32
    for k in (0, 2049, True, 1.5):
        with pytest.raises(ValueError, match="k must"):
            exact_topk(torch.ones(2, 7, device=gpu), k)
    with pytest.raises(ValueError, match="FP32"):
        exact_topk(torch.ones(2, 7, device=gpu, dtype=torch.bfloat16), 3)
