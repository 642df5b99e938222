"""Pins ``oracle.torch_layer`` (the CPU baseline's multi-threaded layer) to the
numpy oracle layer, stage by stage, on the same seeded inputs."""

import numpy as np
import pytest
import torch

from oracle import fp8, kv_fp8, layer as olayer, quantize, sparse_mla as osparse, topk as otopk
from oracle import torch_layer as tlayer


def _inputs(history, queries, seed):
    g = torch.Generator().manual_seed(seed)
    tokens = history + queries
    index_q = torch.randn(queries, 64, 128, generator=g).bfloat16().float()
    index_k = torch.randn(tokens, 128, generator=g).bfloat16().float()
    weights = torch.randn(queries, 64, generator=g) * 0.1
    mla_q = (torch.randn(queries, 128, 576, generator=g) * 0.3).bfloat16().float()
    kv = (torch.randn(tokens, 576, generator=g) * 0.5).bfloat16()
    return index_q, index_k, weights, mla_q, kv


def test_quantize_matches_oracle_bit_for_bit():
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(64, 128, generator=g) * torch.logspace(-3, 3, 64)[:, None]).bfloat16().float()
    values, scale = tlayer.quantize_index(x)
    codes, oscale = quantize.quantize_index(x.numpy())
    assert np.array_equal(scale.numpy().view(np.uint32), oscale.view(np.uint32))
    assert np.array_equal(values.numpy().view(np.uint32), fp8.decode(codes).view(np.uint32))


def test_topk_matches_oracle_exactly_with_ties_and_masks():
    g = torch.Generator().manual_seed(6)
    scores = torch.randint(-4, 5, (6, 700), generator=g).float() * 0.5
    scores[0, ::3] = float("-inf")
    scores[1, :] = 0.0
    scores[2, 10:20] = -0.0
    scores[3, 5] = float("inf")
    for k in (1, 7, 256, 700, 2048):
        values, ids = tlayer.exact_topk(scores, k)
        ovalues, oids = otopk.exact_topk(scores.numpy(), k)
        assert np.array_equal(values.numpy().view(np.uint32), ovalues.view(np.uint32))
        assert np.array_equal(ids.numpy(), oids)


@pytest.mark.parametrize("history,queries,k", [(1024, 8, 256), (3000, 5, 2048)])
def test_layer_matches_oracle_layer(history, queries, k):
    index_q, index_k, weights, mla_q, kv = _inputs(history, queries, seed=history + queries)
    kv_bits = kv.view(torch.int16).numpy().view(np.uint16)
    ocache = olayer.HistoryCache(index_k.numpy(), kv_bits, fp8_records=True)
    records = torch.from_numpy(kv_fp8.decode_records(kv_fp8.encode_records(kv_bits)))
    tcache = tlayer.HistoryCache(index_k, records)
    rows = np.arange(queries)
    oscores, _, oids, oout = olayer.dsa_layer(index_q.numpy(), weights.numpy(), mla_q.numpy(), ocache,
                                              history, rows, k=k)
    tscores, _, tids, tout = tlayer.dsa_layer(index_q, weights, mla_q, tcache, history,
                                              torch.from_numpy(rows), k=k)
    # Logits: the same fp32 formula; only the summation order of the BLAS
    # calls may differ (a few ulps of the largest term of the head sum).
    finite = np.isfinite(oscores)
    assert np.array_equal(finite, np.isfinite(tscores.numpy()))
    scale = np.abs(oscores[finite]).max()
    np.testing.assert_allclose(tscores.numpy()[finite], oscores[finite], rtol=2e-6, atol=2e-6 * scale)
    # Top-k on the torch scores equals the oracle's top-k of the same scores.
    _, ref_ids = otopk.exact_topk(tscores.numpy(), k)
    assert np.array_equal(tids.numpy(), ref_ids)
    # MLA over the same ids: the oracle's fp32 result rounded to bf16.
    _, same_ids_out = osparse.sparse_mla(mla_q.numpy()[rows], ocache.records, tids.numpy(), 576**-0.5)
    expect = fp8.bf16_bits_to_f32(fp8.f32_to_bf16_bits(same_ids_out))
    np.testing.assert_allclose(tout.numpy(), expect, rtol=1.6e-2, atol=1e-5)
    # The selections agree with the oracle's own wherever its scores are not near-ties.
    assert (tids.numpy() == oids).mean() > 0.99
