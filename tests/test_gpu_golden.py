"""The HIP path on the committed golden vectors (tests/golden/dsa_small.npz,
written by the CPU oracle): quantiser, top-k and fp8 KV pack bit-exact; logits
within atol 2e-3 / rtol 1e-3 with exact -inf placement; sparse MLA over the
paged cache within max-abs 2e-2 and cosine >= 0.9999 of the oracle's bf16
output."""

from pathlib import Path

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

GOLD = np.load(Path(__file__).resolve().parent / "golden" / "dsa_small.npz")


def _bf16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


def _fp8(codes, device):
    return torch.from_numpy(np.ascontiguousarray(codes)).to(device).view(torch.float8_e4m3fn)


def test_golden_quantize(gpu):
    from cxldsagr_amd import indexer

    codes, scales = indexer.quantize_index(_bf16(GOLD["quant_x_bits"], gpu))
    assert np.array_equal(codes.view(torch.uint8).cpu().numpy(), GOLD["quant_codes"])
    assert np.array_equal(scales.cpu().numpy().view(np.uint32), GOLD["quant_scales"].view(np.uint32))


def test_golden_logits(gpu):
    from cxldsagr_amd import indexer

    out = indexer.logits(_fp8(GOLD["logits_q"], gpu), _fp8(GOLD["logits_k"], gpu),
                         torch.from_numpy(GOLD["logits_w"]).to(gpu),
                         torch.from_numpy(GOLD["logits_kscale"]).to(gpu),
                         int(GOLD["logits_query_start"])).cpu().numpy()
    want = GOLD["logits_out"]
    finite = np.isfinite(want)
    assert np.array_equal(np.isfinite(out), finite)
    assert np.all(out[~finite] == -np.inf)
    np.testing.assert_allclose(out[finite], want[finite], atol=2e-3, rtol=1e-3)


def test_golden_topk(gpu):
    from cxldsagr_amd import indexer

    values, ids = indexer.exact_topk(torch.from_numpy(GOLD["topk_scores"]).to(gpu), int(GOLD["topk_k"]))
    assert np.array_equal(values.cpu().numpy().view(np.uint32), GOLD["topk_values"].view(np.uint32))
    assert np.array_equal(ids.cpu().numpy(), GOLD["topk_ids"])


def test_golden_kv_pack_and_sparse_mla(gpu):
    from cxldsagr_amd import attention

    table = torch.from_numpy(GOLD["kv_table"]).to(gpu)
    cache = torch.zeros(GOLD["kv_cache"].shape, dtype=torch.uint8, device=gpu)
    attention.pack_kv_fp8(_bf16(GOLD["kv_bits"], gpu), cache, table)
    assert np.array_equal(cache.cpu().numpy(), GOLD["kv_cache"])
    out = attention.sparse_mla_fp8_paged(_bf16(GOLD["mla_q_bits"], gpu), cache, table,
                                         torch.from_numpy(GOLD["mla_ids"]).to(gpu),
                                         float(GOLD["mla_scale"]), n_tokens=GOLD["kv_bits"].shape[0])
    got = out.float().cpu().numpy().astype(np.float64)
    want = (GOLD["mla_out_bits"].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert np.abs(got - want).max() <= 2e-2
    cosine = got.ravel() @ want.ravel() / (np.linalg.norm(got) * np.linalg.norm(want))
    assert cosine >= 0.9999
