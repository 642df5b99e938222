"""A DSA layer step captured in a HIP graph and replayed (the reference tests
CUDA-graph capture of its selection operator, test_selection.py:103-121).

The captured step (fused prologue -> logits -> top-k -> fp8 paged sparse MLA)
is replayed three times; before each replay its outputs are overwritten and
the program runs the same step eagerly, with a synchronisation in between.
Every replay must reproduce the eager outputs bit for bit.
"""

import pytest
import torch

pytestmark = pytest.mark.gpu


# 16384 history columns take the two-part top-k (rows of 8192+ columns).
@pytest.mark.parametrize("history", [4096, 16384])
def test_layer_step_replays_bit_exactly_in_a_graph(gpu, history):
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.workloads import make_layer_inputs

    queries = 64
    inputs = make_layer_inputs(history, queries, seed=521)
    layer = DSALayer(history + queries, device=gpu, kv_format="fp8_paged",
                     page_table=inputs.page_table)
    layer.write_history(inputs.index_k[:history].to(gpu), inputs.kv[:history].to(gpu))
    args = (inputs.index_q.to(gpu), inputs.index_k[history:].to(gpu), inputs.weights.to(gpu),
            inputs.mla_q.to(gpu), inputs.kv[history:].to(gpu))

    def step():
        layer.written = history  # the same step again: same cache rows, same inputs
        out, selection = layer.forward(*args)
        return out, selection.token_ids

    out_eager, ids_eager = (t.clone() for t in step())
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream's kind of stream
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_graph, ids_graph = step()
    torch.cuda.synchronize()

    for replay in range(3):
        print(f"replay {replay}", flush=True)
        out_graph.fill_(float("nan"))
        ids_graph.fill_(-7)
        again_out, again_ids = step()  # the program's own eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(again_out.view(torch.int16), out_eager.view(torch.int16))
        assert torch.equal(again_ids, ids_eager)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_graph.view(torch.int16), out_eager.view(torch.int16)), replay
        assert torch.equal(ids_graph, ids_eager), replay


def test_layer_step_from_gemm_outputs_replays_bit_exactly_in_a_graph(gpu):
    """The same for the layer step from the indexer's GEMM outputs (producer
    launch: LayerNorm, RoPE, quantisation, fold, cache writes; then logits,
    top-k and sparse MLA)."""
    from cxldsagr_amd import projections
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.workloads import make_layer_inputs

    history, queries = 16384, 64
    inputs = make_layer_inputs(history, queries, seed=734)
    layer = DSALayer(history + queries, device=gpu, kv_format="fp8_paged",
                     page_table=inputs.page_table)
    layer.write_history(inputs.index_k[:history].to(gpu), inputs.kv[:history].to(gpu))
    g = torch.Generator().manual_seed(9)
    projection = projections.IndexerProjection(
        torch.zeros(64 * 128, 16, dtype=torch.bfloat16, device=gpu),
        torch.zeros(128, 16, dtype=torch.bfloat16, device=gpu),
        torch.zeros(64, 16, device=gpu), (1 + 0.1 * torch.randn(128, generator=g)).to(gpu),
        (0.1 * torch.randn(128, generator=g)).to(gpu), projections.rotary_frequencies().to(gpu))
    positions = torch.arange(history, history + queries, dtype=torch.float32, device=gpu)
    projected = projections.IndexProjected(
        inputs.index_q.to(gpu), inputs.index_k[history:].to(gpu), inputs.weights.to(gpu) * 8,
        projections.rotary_table(positions, projection.frequencies))
    mla_q, kv = inputs.mla_q.to(gpu), inputs.kv[history:].to(gpu)

    def step():
        layer.written = history
        out, selection = layer.forward_projected(projection, projected, mla_q, kv)
        return out, selection.token_ids

    out_eager, ids_eager = (t.clone() for t in step())
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_graph, ids_graph = step()
    torch.cuda.synchronize()
    for replay in range(3):
        print(f"replay {replay}", flush=True)
        out_graph.fill_(float("nan"))
        ids_graph.fill_(-7)
        layer.index_keys[history:].zero_()  # the producer rewrites the new rows
        again_out, again_ids = step()
        torch.cuda.synchronize()
        assert torch.equal(again_out.view(torch.int16), out_eager.view(torch.int16))
        assert torch.equal(again_ids, ids_eager)
        layer.index_keys[history:].zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_graph.view(torch.int16), out_eager.view(torch.int16)), replay
        assert torch.equal(ids_graph, ids_eager), replay
