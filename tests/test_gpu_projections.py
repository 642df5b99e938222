"""Indexer input producers on the GPU (``dsa_index_producer_fp8``) against the
CPU oracle ``oracle.projections`` (pinned in ``tests/test_oracle_projections.py``).

Bit-exact: index Q and K codes and scales, the folded head weights, the
index-cache rows written in place and the fp8 KV records. The partial folded
queries are checked through the logits kernel, which must write the same
bits with and without them. The layer step from GEMM outputs
(``DSALayer.forward_projected``) is compared with the plain ``forward`` given
the oracle's post-RoPE bf16 indexer inputs.
"""

import numpy as np
import pytest
import torch

from oracle import kv_fp8 as okv
from oracle import projections as oproj

pytestmark = pytest.mark.gpu


def _bits(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def _inputs(tokens, seed, start=65536):
    from cxldsagr_amd.projections import rotary_frequencies, rotary_table

    g = torch.Generator().manual_seed(seed)
    q_proj = torch.randn(tokens, 64, 128, generator=g).bfloat16()
    k_proj = (torch.randn(tokens, 128, generator=g) * 2 + 0.3).bfloat16()
    head = torch.randn(tokens, 64, generator=g) * 4
    norm_w = 1 + 0.1 * torch.randn(128, generator=g)
    norm_b = 0.1 * torch.randn(128, generator=g)
    positions = torch.arange(start, start + tokens, dtype=torch.float32)
    table = rotary_table(positions, rotary_frequencies())
    return q_proj, k_proj, head, norm_w, norm_b, table


def _oracle(q_proj, k_proj, head, norm_w, norm_b, table, rows=None):
    rows = np.arange(len(q_proj)) if rows is None else rows
    return oproj.index_producer(_bits(q_proj), _bits(k_proj), norm_w.numpy(), norm_b.numpy(),
                                1e-6, table.numpy(), rows, head.numpy())


def _check(got, ref):
    q8, qs, w, k8, ks = got[:5]
    rq8, rqs, rk8, rks, rw = ref
    np.testing.assert_array_equal(q8.view(torch.uint8).cpu().numpy(), rq8)
    np.testing.assert_array_equal(qs.cpu().numpy().view(np.uint32), rqs.view(np.uint32))
    np.testing.assert_array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32))
    np.testing.assert_array_equal(k8.view(torch.uint8).cpu().numpy(), rk8)
    np.testing.assert_array_equal(ks.cpu().numpy().view(np.uint32), rks.view(np.uint32))


@pytest.mark.parametrize("tokens", [1, 37, 128, 512])
def test_producer_matches_oracle(gpu, tokens):
    from cxldsagr_amd.projections import index_producer

    q_proj, k_proj, head, norm_w, norm_b, table = _inputs(tokens, seed=tokens)
    got = index_producer(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), norm_w.to(gpu),
                         norm_b.to(gpu), 1e-6, table.to(gpu))
    torch.cuda.synchronize()
    _check(got, _oracle(q_proj, k_proj, head, norm_w, norm_b, table))


def test_producer_many_k_rows_exercise_layer_norm_rounding(gpu):
    """16,384 index-K rows with a large common offset (LayerNorm subtracts a
    mean far from zero, so its rounding matters): the codes stay bit-exact."""
    from cxldsagr_amd.projections import index_producer

    tokens = 16384
    q_proj, k_proj, head, norm_w, norm_b, table = _inputs(tokens, seed=5, start=0)
    k_proj = (k_proj.float() * 0.01 + 37.0).bfloat16()
    got = index_producer(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), norm_w.to(gpu),
                         norm_b.to(gpu), 1e-6, table.to(gpu))
    torch.cuda.synchronize()
    _check(got, _oracle(q_proj, k_proj, head, norm_w, norm_b, table))


def test_rope_rows_select_table_rows_and_flag_out_of_range(gpu):
    from cxldsagr_amd.projections import index_producer

    tokens = 9
    q_proj, k_proj, head, norm_w, norm_b, _ = _inputs(tokens, seed=2)
    _, _, _, _, _, table = _inputs(50, seed=3, start=1000)
    rows = np.array([49, 0, 7, 7, 30, 2, 11, 48, 5], np.int32)
    status = torch.zeros(1, dtype=torch.int32, device=gpu)
    got = index_producer(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), norm_w.to(gpu),
                         norm_b.to(gpu), 1e-6, table.to(gpu), torch.from_numpy(rows).to(gpu),
                         status=status)
    torch.cuda.synchronize()
    assert status.item() == 0
    _check(got, _oracle(q_proj, k_proj, head, norm_w, norm_b, table, rows))

    bad = rows.copy()
    bad[3] = 50      # past the table: flagged, row 0 used
    got = index_producer(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), norm_w.to(gpu),
                         norm_b.to(gpu), 1e-6, table.to(gpu), torch.from_numpy(bad).to(gpu),
                         status=status)
    torch.cuda.synchronize()
    assert status.item() & 2
    bad[3] = 0
    _check(got, _oracle(q_proj, k_proj, head, norm_w, norm_b, table, bad))


def test_producer_writes_cache_rows_kv_records_and_q_fold(gpu):
    """In-place index-cache rows and fp8 KV records; the partial folded
    queries give the same logits bits as the kernel's own."""
    from cxldsagr_amd import indexer
    from cxldsagr_amd.projections import index_producer

    history, tokens = 300, 40
    q_proj, k_proj, head, norm_w, norm_b, table = _inputs(history + tokens, seed=4, start=0)
    keys = torch.zeros((history + tokens, 128), dtype=torch.float8_e4m3fn, device=gpu)
    scales = torch.zeros(history + tokens, dtype=torch.float32, device=gpu)
    g = torch.Generator().manual_seed(9)
    kv = torch.randn(history + tokens, 576, generator=g).bfloat16()
    pages = (history + tokens + 63) // 64
    page_table = torch.randperm(pages, generator=g).int().to(gpu)
    cache = torch.zeros((pages, 64, 656), dtype=torch.uint8, device=gpu)
    # History first (no q fold), then the new tokens at offset `history`.
    for lo, hi, fold in ((0, history, False), (history, history + tokens, True)):
        out = index_producer(q_proj[lo:hi].to(gpu), k_proj[lo:hi].to(gpu), head[lo:hi].to(gpu),
                             norm_w.to(gpu), norm_b.to(gpu), 1e-6, table[lo:hi].to(gpu),
                             index_keys=keys[lo:hi], index_scales=scales[lo:hi], q_fold=fold,
                             kv=kv[lo:hi].to(gpu), kv_cache=cache, page_table=page_table,
                             token_offset=lo)
    torch.cuda.synchronize()
    ref = _oracle(q_proj, k_proj, head, norm_w, norm_b, table)
    np.testing.assert_array_equal(keys.view(torch.uint8).cpu().numpy(), ref[2])
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), ref[3].view(np.uint32))
    records = okv.encode_records(_bits(kv))
    flat = cache.view(-1, 656).cpu().numpy()
    rows = okv.physical_rows(page_table.cpu().numpy(), history + tokens)
    np.testing.assert_array_equal(flat[rows], records)

    q8, _, w, _, _, q_fold = out
    a = indexer.logits(q8, keys, w, scales, history, _pad_to_stride=True)
    b = indexer.logits(q8, keys, w, scales, history, _pad_to_stride=True, _q_fold=q_fold)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


@pytest.mark.parametrize("kv_format", ["fp8_paged", "bf16"])
def test_layer_forward_projected_equals_forward(gpu, kv_format):
    """The layer step from GEMM outputs equals ``forward``, bit for bit, on
    the oracle's post-RoPE bf16 indexer inputs and the head weights scaled by
    64**-0.5 and 128**-0.5 (the fold multiplies by the power-of-two q-scale
    in between, which commutes exactly with the roundings). The candidate
    top-k's floors, estimated in the producer launch from the queries it
    rotates, equal those of forward's prologue bit for bit."""
    from cxldsagr_amd import indexer
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.projections import IndexProjected, IndexerProjection, rotary_frequencies
    from cxldsagr_amd.workloads import make_layer_inputs

    history, queries = 16384, 128  # past the 8192 visible keys below which rows get no floor
    inputs = make_layer_inputs(history, queries, seed=11)
    tokens = history + queries
    q_proj, k_proj, head, norm_w, norm_b, table = _inputs(queries, seed=12, start=history)
    kw = dict(device=gpu, kv_format=kv_format, page_table=inputs.page_table)
    a, b = DSALayer(tokens, **kw), DSALayer(tokens, **kw)
    for layer in (a, b):
        layer.write_history(inputs.index_k[:history].to(gpu), inputs.kv[:history].to(gpu))
    projection = IndexerProjection(torch.zeros(8192, 16, dtype=torch.bfloat16, device=gpu),
                                   torch.zeros(128, 16, dtype=torch.bfloat16, device=gpu),
                                   torch.zeros(64, 16, device=gpu), norm_w.to(gpu),
                                   norm_b.to(gpu), rotary_frequencies().to(gpu))
    projected = IndexProjected(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), table.to(gpu))
    mla_q, kv = inputs.mla_q.to(gpu), inputs.kv[history:].to(gpu)
    out_a, sel_a = a.forward_projected(projection, projected, mla_q, kv)
    floors_a = indexer.select_floors_buffer(gpu, queries, tokens).clone()

    # The same step through forward(): bf16 index Q/K after RoPE from the
    # oracle, weights scaled so that their fold equals the producer's.
    cos, sin = table.numpy()[:, :32], table.numpy()[:, 32:]
    index_q = oproj.index_q(_bits(q_proj), cos, sin)
    index_k = oproj.index_k(_bits(k_proj), norm_w.numpy(), norm_b.numpy(), 1e-6, cos, sin)
    weights = (head.numpy() * oproj.INV_SQRT_HEADS).astype(np.float32)
    weights = (weights * oproj.INV_SQRT_DIM).astype(np.float32)
    to_bf16 = lambda x: torch.from_numpy(x).bfloat16().to(gpu)  # noqa: E731 (exact: bf16 values)
    out_b, sel_b = b.forward(to_bf16(index_q), to_bf16(index_k), torch.from_numpy(weights).to(gpu),
                             mla_q, kv)
    floors_b = indexer.select_floors_buffer(gpu, queries, tokens).clone()
    torch.cuda.synchronize()
    assert (floors_a != 0).all()
    assert torch.equal(floors_a, floors_b)
    assert torch.equal(a.index_keys.view(torch.uint8), b.index_keys.view(torch.uint8))
    if kv_format == "fp8_paged":
        assert torch.equal(a.kv_cache, b.kv_cache)
    assert torch.equal(sel_a.token_ids, sel_b.token_ids)
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))


def test_projection_gemms_then_producer(gpu):
    """IndexerProjection.project (library GEMMs: index_wq on qr, index_wk on x,
    weights_proj on x in fp32, and the RoPE table of the positions) then
    produce: the producer's outputs equal the oracle applied to the GEMM
    outputs project returned."""
    from cxldsagr_amd.projections import IndexerProjection, rotary_frequencies

    tokens, dim, q_lora = 48, 512, 256
    g = torch.Generator().manual_seed(21)
    x = torch.randn(tokens, dim, generator=g).bfloat16().to(gpu)
    qr = torch.randn(tokens, q_lora, generator=g).bfloat16().to(gpu)
    projection = IndexerProjection(
        (torch.randn(64 * 128, q_lora, generator=g) / 16).bfloat16().to(gpu),
        (torch.randn(128, dim, generator=g) / 16).bfloat16().to(gpu),
        (torch.randn(64, dim, generator=g) / 16).to(gpu),
        (1 + 0.1 * torch.randn(128, generator=g)).to(gpu), (0.1 * torch.randn(128, generator=g)).to(gpu),
        rotary_frequencies().to(gpu))
    positions = torch.arange(1000, 1000 + tokens, dtype=torch.float32, device=gpu)
    projected = projection.project(x, qr, positions)
    assert tuple(projected.q_proj.shape) == (tokens, 64, 128)
    assert tuple(projected.k_proj.shape) == (tokens, 128)
    assert projected.head_logits.dtype == torch.float32
    got = projection.produce(projected)
    torch.cuda.synchronize()
    ref = oproj.index_producer(_bits(projected.q_proj.cpu()), _bits(projected.k_proj.cpu()),
                               projection.norm_weight.cpu().numpy(),
                               projection.norm_bias.cpu().numpy(), 1e-6,
                               projected.cos_sin.cpu().numpy(), np.arange(tokens),
                               projected.head_logits.cpu().numpy())
    _check(got, ref)
    # The GEMMs are the reference's: F.linear on the same operands.
    expect_q = torch.nn.functional.linear(qr, projection.index_wq).view(tokens, 64, 128)
    assert torch.equal(projected.q_proj, expect_q)
    expect_w = torch.nn.functional.linear(x.float(), projection.weights_proj)
    assert torch.equal(projected.head_logits, expect_w)


def test_producer_floors_follow_rope_rows(gpu):
    """The producer's floor blocks rotate each query with its own RoPE table
    row (``rope_rows``): their floors equal those the layer prologue
    estimates from the oracle's rotated queries and the matching weights."""
    from cxldsagr_amd import indexer
    from cxldsagr_amd.layer import index_prologue
    from cxldsagr_amd.projections import index_producer

    history, tokens = 16384, 64
    q_proj, k_proj, head, norm_w, norm_b, _ = _inputs(tokens, seed=31)
    _, _, _, _, _, table = _inputs(200, seed=32, start=5000)
    rows = torch.randperm(200, generator=torch.Generator().manual_seed(33))[:tokens].int()
    g = torch.Generator().manual_seed(34)
    history_keys = torch.randn(history, 128, generator=g).bfloat16().to(gpu)
    caches = []
    for _ in range(2):
        keys = torch.zeros((history + tokens, 128), dtype=torch.float8_e4m3fn, device=gpu)
        scales = torch.zeros(history + tokens, dtype=torch.float32, device=gpu)
        indexer.quantize_into(history_keys, keys[:history], scales[:history])
        caches.append((keys, scales))

    floors_a = torch.zeros((tokens, 2), dtype=torch.int32, device=gpu)
    keys, scales = caches[0]
    index_producer(q_proj.to(gpu), k_proj.to(gpu), head.to(gpu), norm_w.to(gpu), norm_b.to(gpu),
                   1e-6, table.to(gpu), rows.to(gpu), index_keys=keys[history:],
                   index_scales=scales[history:], token_offset=history, floors=floors_a,
                   key_cache=keys, key_cache_scales=scales)

    picked = table.numpy()[rows.numpy()]
    index_q = oproj.index_q(_bits(q_proj), picked[:, :32], picked[:, 32:])
    weights = (head.numpy() * oproj.INV_SQRT_HEADS).astype(np.float32)
    weights = (weights * oproj.INV_SQRT_DIM).astype(np.float32)
    floors_b = torch.zeros((tokens, 2), dtype=torch.int32, device=gpu)
    keys, scales = caches[1]
    index_prologue(torch.from_numpy(index_q).bfloat16().to(gpu), k_proj.to(gpu),
                   torch.from_numpy(weights).to(gpu), keys, scales, history, 2048, floors_b)
    torch.cuda.synchronize()
    assert (floors_a != 0).all()
    assert torch.equal(floors_a, floors_b)
