"""The flat operator namespace keeps the reference's names, argument order,
argument kinds and defaults (CPU; nothing is launched).

Reference signatures: quantization.py:63, echo.py:299, selection.py:62,
device_only/mla.py:90, offload/mla.py:12, kv_transfer.py:21. Extra
keyword-only arguments after the reference's own are allowed.
"""

import inspect

import pytest

from cxldsagr_amd import ops

P = inspect.Parameter
REFERENCE = {
    "quantize_index": [("x", P.POSITIONAL_OR_KEYWORD, P.empty), ("scale_fmt", P.POSITIONAL_OR_KEYWORD, "ue8m0")],
    "logits": [
        ("q", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("k", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("weights", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("kscale", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("query_start", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("prefetch", P.POSITIONAL_OR_KEYWORD, None),
        ("_bounds", P.KEYWORD_ONLY, None),
        ("_pad_to_stride", P.KEYWORD_ONLY, False),
    ],
    "exact_topk": [("scores", P.POSITIONAL_OR_KEYWORD, P.empty), ("k", P.POSITIONAL_OR_KEYWORD, P.empty)],
    "sparse_mla": [
        ("q", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("kv", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("indices", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("scale", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("value_dim", P.POSITIONAL_OR_KEYWORD, 512),
    ],
    "sparse_mla_from_pool": [
        ("q", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("records", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("physical_indices", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("scale", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("value_dim", P.POSITIONAL_OR_KEYWORD, 512),
    ],
    "gather_host_records": [
        ("host", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("device", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("host_ids", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("device_ids", P.POSITIONAL_OR_KEYWORD, P.empty),
        ("max_ctas", P.KEYWORD_ONLY, None),
        ("valid_count", P.KEYWORD_ONLY, None),
    ],
}


@pytest.mark.parametrize("name", sorted(REFERENCE))
def test_reference_signature_is_kept(name):
    params = list(inspect.signature(getattr(ops, name)).parameters.values())
    want = REFERENCE[name]
    got = [(p.name, p.kind, p.default) for p in params[: len(want)]]
    assert got == want
    # Anything beyond the reference's parameters is keyword-only with a default.
    for extra in params[len(want):]:
        assert extra.kind == P.KEYWORD_ONLY and extra.default is not P.empty, extra


def test_every_export_is_present():
    for name in ops.__all__:
        assert callable(getattr(ops, name)), name
