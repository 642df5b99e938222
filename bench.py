#!/usr/bin/env python3
"""Benchmark: one DSA prefill layer at 64K history + 128 query tokens on one MI355X.

A step is one full layer through the HIP kernels, with every input already
resident in HBM: quantise the indexer Q, fold its scales into the head
weights, quantise the 128 new index keys into the resident index cache, fp8
logits over 65,664 keys with the causal tail, exact top-2048, pack the 128
new KV records into the fp8 paged cache, sparse MLA (128 heads, 2048
selected, 656-byte fp8 records). Workload = BASELINE configs 1 and 2 (same
seed, seeded synthetic inputs of the DeepSeek-V3.2 shapes).

Prints one JSON line. ``value`` is microseconds per layer (lower is better).
``roofline`` is for the kernel with the largest share of the step, timed with
HIP events on the stream it is launched on; ``kernels`` lists every stage.
``cpu_baseline`` times the torch CPU restatement of the same layer
(``oracle/torch_layer.py``, pinned to the numpy oracle) on all 128 query rows
with torch's intra-op threads on this process's cores.
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAKS = {  # MI355X published dense peaks
    "hbm_GBps": 8000.0,
    "fp8_TFLOPs": 5000.0,
    "bf16_TFLOPs": 2500.0,
}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--history", type=int, default=65536)
    p.add_argument("--queries", type=int, default=128)
    p.add_argument("--seed", type=int, default=947)
    p.add_argument("--cpu-rows", type=int, default=128,
                   help="query rows of the CPU baseline sample (scaled to all rows)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--no-config4", action="store_true",
                   help="skip the compact config-4 layer time of the default line")
    p.add_argument("--no-config3", action="store_true",
                   help="skip the compact config-3 layer times of the default line")
    p.add_argument("--only", choices=["layer", "logits", "topk", "mla", "producer"], default=None,
                   help="time only one stage (for profiler runs)")
    p.add_argument("--copy-calibration-mib", type=int, default=0,
                   help="first run one plain device copy of this many MiB (scales PMC byte "
                        "counters in profiler runs)")
    p.add_argument("--config", type=int, choices=[1, 3, 4], default=1,
                   help="1: the headline layer (configs 1+2, default); 3: GR multi-user recall "
                        "over a pinned-host token pool; 4: long-context stress, fp8 and bf16 KV")
    p.add_argument("--users", type=int, default=16, help="config 3: users")
    return p.parse_args()


def spin_up(torch, fn, seconds=0.2):
    """Run fn() (untimed) for a fixed wall time before the warm-up steps: the
    GPU needs some tens of milliseconds of load to reach its steady clock, and
    a handful of warm-up steps alone leave the first timed steps ~8 % slow."""
    import time

    torch.cuda.synchronize()
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end:
        for _ in range(16):
            fn()
        torch.cuda.synchronize()


def event_time_us(torch, fn, iters):
    """Average duration of fn() over iters launches, HIP events on the current stream."""
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for _ in range(iters):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1e3 / iters


def select_workspace(rows, tokens, device):
    import ctypes

    import torch

    from cxldsagr_amd import _native

    needed = ctypes.c_int64()
    _native.call("dsa_indexer_select_workspace_bytes", rows, tokens, 0, ctypes.byref(needed))
    return torch.empty(needed.value, dtype=torch.uint8, device=device)


def indexer_stage_calls(layer, tokens, topk, q8, folded, q_fold, workspace):
    """The launches of the layer's indexer step after its prologue (which
    writes the per-row floors into ``workspace``) as separate calls: the
    logits kernel writing only the candidates at or above the floors, and the
    top-k of the candidates. Returns (logits_fn, topk_fn, ids)."""
    import torch

    from cxldsagr_amd import _native, indexer

    device = q8.device
    rows, width = len(q8), indexer.padded_columns(tokens)
    scores = torch.empty(rows, width, device=device)
    count = min(topk, tokens)
    ids = torch.empty(rows, count, dtype=torch.int32, device=device)
    values = torch.empty(rows, count, device=device)
    keys, kscale = layer.index_keys[:tokens], layer.index_scales[:tokens]
    history = tokens - rows
    head = (_native.ptr(q8), _native.ptr(keys), _native.ptr(folded), _native.ptr(kscale), None,
            None, history, rows, tokens)

    def logits_fn():
        _native.call("dsa_indexer_logits_fp8_emit", *head, width, _native.ptr(q_fold),
                     _native.ptr(scores), 0, _native.ptr(workspace), workspace.numel(),
                     _native.stream_of(device))

    def topk_fn():
        _native.call("dsa_indexer_emit_topk", *head, _native.ptr(q_fold), _native.ptr(scores), topk,
                     _native.ptr(values), _native.ptr(ids), count, 0, _native.ptr(workspace),
                     workspace.numel(), _native.stream_of(device))

    return logits_fn, topk_fn, ids


# "marker" is an empty bracket: two events recorded back to back, the cost
# one event marker adds to each stage interval.
STAGES = ("marker", "prologue", "logits", "topk", "sparse_mla")


def in_layer_stage_us(torch, layer, history, tokens, topk, iters, args):
    """Average duration of each stage of the layer step, from HIP events recorded
    between its launches on the current stream (the same launches, in the same
    order, as DSALayer.forward; the per-row floors are part of the prologue
    launch), after an empty bracket that measures what one event marker adds
    to a stage. Also returns the candidate keys the indexer step listed and
    the key splits that spilled."""
    index_q, index_k, weights, mla_q, kv = args
    fused = layer._fused_prologue_applies(index_q, index_k, weights, kv)
    stream = torch.cuda.current_stream()
    marks = [[torch.cuda.Event(enable_timing=True) for _ in range(len(STAGES) + 1)]
             for _ in range(iters)]
    rows = len(index_q)
    workspace = select_workspace(rows, tokens, layer.device)
    floors = workspace[:8 * rows].view(torch.int32).view(rows, 2)

    from cxldsagr_amd.layer import index_prologue

    def prologue():
        if fused:
            return layer._prologue(index_q, index_k, weights, kv, history, floors)
        # bf16 records: the prologue without the KV pack, then the record copy.
        out = index_prologue(index_q, index_k, weights, layer.index_keys, layer.index_scales,
                             history, topk, floors)
        layer._append_kv(kv, history)
        return out

    layer.written = history
    q8, folded, q_fold = prologue()
    logits_fn, topk_fn, ids = indexer_stage_calls(
        layer, tokens, topk, q8, folded, q_fold, workspace)
    torch.cuda.synchronize()
    for ev in marks:
        layer.written = history
        ev[0].record(stream)
        ev[1].record(stream)
        prologue()
        ev[2].record(stream)
        logits_fn()
        ev[3].record(stream)
        topk_fn()
        ev[4].record(stream)
        layer._attend(mla_q, ids, tokens)
        ev[5].record(stream)
    torch.cuda.synchronize()
    # Candidates listed per row (records [rows][splits][2] after the floors).
    records_at = (8 * rows + 255) // 256 * 256
    width = (tokens + 255) // 256 * 256
    cus = torch.cuda.get_device_properties(layer.device).multi_processor_count
    qgroups = (rows + 15) // 16
    splits = max(1, (cus + qgroups - 1) // qgroups)
    per = ((width + splits - 1) // splits + 127) // 128 * 128
    splits = (width + per - 1) // per
    splits = (splits + 7) // 8 * 8 if splits >= 8 else splits
    rec = workspace[records_at:records_at + rows * splits * 8].view(torch.int32).view(rows, splits, 2)
    live = [sp for sp in range(splits) if sp * per < tokens]
    candidates = int(rec[:, live, 0].sum().item())
    spilled = int((rec[:, live, 1] != 0x7FFFFFFF).sum().item())
    times = {name: sum(ev[i].elapsed_time(ev[i + 1]) for ev in marks) * 1e3 / iters
             for i, name in enumerate(STAGES)}
    return times, candidates, spilled


def cpu_baseline(inputs, rows_sample, topk):
    """The same layer on the host: ``oracle.torch_layer`` (torch CPU kernels,
    intra-op threads on every core of this process's affinity, capped by
    OMP_NUM_THREADS where the environment sets a CPU share)."""
    import numpy as np
    import torch

    from oracle import kv_fp8
    from oracle import torch_layer as tlayer

    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(max(1, threads))
    history, queries = inputs.history, inputs.queries
    index_q = inputs.index_q.float().cpu()
    weights = inputs.weights.float().cpu()
    mla_q = inputs.mla_q.float().cpu()
    kv_bits = inputs.kv.cpu().view(torch.int16).numpy().view(np.uint16)
    records = torch.from_numpy(kv_fp8.decode_records(kv_fp8.encode_records(kv_bits)))
    cache = tlayer.HistoryCache(inputs.index_k.float().cpu(), records)  # resident, as on the GPU
    rows_sample = min(max(1, rows_sample), queries)
    rows = torch.from_numpy(np.linspace(0, queries - 1, rows_sample).round().astype(np.int64))
    tlayer.dsa_layer(index_q, weights, mla_q, cache, history, rows[:1], k=topk)  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter_ns()
        tlayer.dsa_layer(index_q, weights, mla_q, cache, history, rows, k=topk)
        times.append((time.perf_counter_ns() - t0) / 1e3)
    per_layer = sorted(times)[1] * queries / len(rows)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    scaled = "" if len(rows) == queries else f", scaled x{queries / len(rows):g}"
    return {
        "value": round(per_layer, 1),
        "unit": "us/layer",
        "cores": int(torch.get_num_threads()),
        "kind": "port",
        "sample": f"torch CPU restatement of the oracle layer (A1 Q quantise, A4 logits, A6 "
                  f"top-k, A7 MLA over dequantised fp8 records), {len(rows)} of {queries} query "
                  f"rows, median of 3{scaled}; resident K/KV caches prebuilt as on the GPU",
        "cpu": cpu_model,
        "affinity": len(os.sched_getaffinity(0)),
    }


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported here "
              "(the DSA layer step is measured on one GPU's share of the work)",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from cxldsagr_amd import attention, indexer
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.workloads import make_layer_inputs

    if args.config == 3:
        return bench_config3(args)
    if args.config == 4:
        return bench_config4(args)
    device = torch.device("cuda", 0)
    history, queries, topk = args.history, args.queries, 2048
    tokens = history + queries
    inputs = make_layer_inputs(history, queries, seed=args.seed)
    layer = DSALayer(tokens, device=device, kv_format="fp8_paged", page_table=inputs.page_table)
    layer.write_history(inputs.index_k[:history].to(device), inputs.kv[:history].to(device))
    index_q = inputs.index_q.to(device)
    index_k_new = inputs.index_k[history:].to(device).contiguous()
    weights = inputs.weights.to(device)
    mla_q = inputs.mla_q.to(device)
    kv_new = inputs.kv[history:].to(device).contiguous()

    def step():
        layer.written = history
        return layer.forward(index_q, index_k_new, weights, mla_q, kv_new)

    # Intermediates for per-stage timing (same values the step produces).
    out, selection = step()
    q8, _, w_eff = indexer.quantize_index_folded(index_q, weights)
    keys, kscale = layer.index_keys[:tokens], layer.index_scales[:tokens]
    scores = indexer.logits(q8, keys, w_eff, kscale, history, _pad_to_stride=True)
    _, ids = indexer.exact_topk(scores, topk)
    torch.cuda.synchronize()

    # The same layer from the indexer's GEMM outputs: the producer launch (K
    # LayerNorm, RoPE of Q and K, quantisation, weight fold, index-cache
    # write, KV pack) in place of the prologue. GEMM outputs are stand-ins of
    # the right shapes (the index Q/K of the workload, head logits from its
    # weights) with a unit LayerNorm and the YaRN table of the positions.
    from cxldsagr_amd import projections

    projection = projections.IndexerProjection(
        torch.zeros(64 * 128, 16, dtype=torch.bfloat16, device=device),
        torch.zeros(128, 16, dtype=torch.bfloat16, device=device),
        torch.zeros(64, 16, device=device), torch.ones(128, device=device),
        torch.zeros(128, device=device), projections.rotary_frequencies().to(device))
    positions = torch.arange(history, tokens, dtype=torch.float32, device=device)
    projected = projections.IndexProjected(index_q, index_k_new, weights * 8.0,
                                           projections.rotary_table(positions,
                                                                    projection.frequencies))

    def projected_step():
        layer.written = history
        return layer.forward_projected(projection, projected, mla_q, kv_new)

    def producer_stage():
        return projection.produce(projected, index_keys=layer.index_keys[history:tokens],
                                  index_scales=layer.index_scales[history:tokens], q_fold=True,
                                  kv=kv_new, kv_cache=layer.kv_cache, page_table=layer.page_table,
                                  token_offset=history)

    # Isolated stages: the layer's indexer step (floors, candidate logits,
    # top-k of the candidates) as one call; the earlier fused step that writes
    # every score and counts its digits, and the unfused logits and top-k,
    # beside it.
    stages = {
        "index_producer": producer_stage,
        "quantize_q": lambda: indexer.quantize_index_folded(index_q, weights),
        "select_topk": lambda: indexer.select_topk(q8, keys, w_eff, kscale, history, topk),
        "logits_topk_counted": lambda: indexer.logits_topk(q8, keys, w_eff, kscale, history, topk),
        "logits_unfused": lambda: indexer.logits(q8, keys, w_eff, kscale, history,
                                                 _pad_to_stride=True),
        "topk_unfused": lambda: indexer.exact_topk(scores, topk),
        "pack_kv": lambda: attention.pack_kv_fp8(kv_new, layer.kv_cache, layer.page_table,
                                                 token_offset=history),
        "sparse_mla": lambda: attention.sparse_mla_fp8_paged(
            mla_q, layer.kv_cache, layer.page_table, ids, layer.scale, n_tokens=tokens),
    }
    if args.copy_calibration_mib:
        src = torch.ones(args.copy_calibration_mib << 18, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    if args.only is not None:
        fn = step if args.only == "layer" else stages[{"mla": "sparse_mla", "topk": "select_topk", "logits": "logits_unfused", "producer": "index_producer"}.get(args.only, args.only)]
        for _ in range(args.warmup):
            fn()
        us = event_time_us(torch, fn, args.steps)
        print(json.dumps({"only": args.only, "us": round(us, 2), "steps": args.steps}))
        return

    spin_up(torch, step)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    layer_us = event_time_us(torch, step, args.steps)

    isolated_us = {name: event_time_us(torch, fn, args.steps) for name, fn in stages.items()}
    projected_layer_us = event_time_us(torch, projected_step, args.steps)
    step()  # leave the layer as the plain step left it
    torch.cuda.synchronize()
    in_layer, candidates, spilled = in_layer_stage_us(
        torch, layer, history, tokens, topk, args.steps,
        (index_q, index_k_new, weights, mla_q, kv_new))
    # Kernel figures are the launches inside the layer step (the clock of the
    # timed region), each stage's event interval less the cost of one marker
    # (the empty bracket); the isolated stage loops are reported beside them.
    kernel_us = dict(isolated_us)
    kernel_us.update({name: us - in_layer["marker"] for name, us in in_layer.items()})
    kernel_us["marker"] = in_layer["marker"]
    pairs = queries * history + queries * (queries + 1) // 2
    logits_flop = 2 * 64 * 128 * pairs
    mla_flop = 2 * queries * topk * 128 * (576 + 512)
    gather_bytes = queries * topk * 656
    # The top-k of the candidates reads the listed composite keys (8 B each)
    # and writes 8 B per selected (value, id).
    topk_bytes = candidates * 8 + queries * topk * 8
    producer_bytes = ((queries * 64 + queries) * (256 + 128 + 4 + 256) + queries * 64 * 8
                      + queries * 4 * 128 * 4 + queries * (1152 + 656))
    kernels = {
        "logits": {
            "us": round(kernel_us["logits"], 2),
            "TFLOPs": round(logits_flop / kernel_us["logits"] / 1e6, 1),
            "frac_fp8_peak": round(logits_flop / kernel_us["logits"] / 1e6 / PEAKS["fp8_TFLOPs"], 4),
        },
        "topk": {
            "us": round(kernel_us["topk"], 2),
            "GBps": round(topk_bytes / kernel_us["topk"] / 1e3, 1),
            "candidates": candidates,
            "spilled_splits": spilled,
        },
        "sparse_mla": {
            "us": round(kernel_us["sparse_mla"], 2),
            "TFLOPs": round(mla_flop / kernel_us["sparse_mla"] / 1e6, 1),
            "frac_bf16_peak": round(mla_flop / kernel_us["sparse_mla"] / 1e6 / PEAKS["bf16_TFLOPs"], 4),
            "gather_GBps": round(gather_bytes / kernel_us["sparse_mla"] / 1e3, 1),
            "gather_frac_hbm": round(gather_bytes / kernel_us["sparse_mla"] / 1e3 / PEAKS["hbm_GBps"], 4),
        },
        # One launch: Q quantisation + weight fold, the new index K into the
        # cache, the new KV records packed, and the candidate top-k's per-row
        # floors.
        "prologue": {"us": round(kernel_us["prologue"], 2), "with_floors": True},
        # Each stage's event interval before the marker is taken off.
        "stage_us": {name: round(in_layer[name], 2) for name in STAGES[1:]},
        # Algorithmic bytes of the producer launch: per 128-value row 256 B in,
        # 128 B codes + 4 B scale out, 256 B of its RoPE row; per Q row 4 B head
        # logit in + 4 B weight out; the partial folded queries; per KV token
        # 1152 B in + 656 B out.
        "index_producer": {
            "us": round(isolated_us["index_producer"], 2),
            "GBps": round(producer_bytes / isolated_us["index_producer"] / 1e3, 1),
            "bytes": producer_bytes,
        },
        "isolated_us": {name: round(us, 2) for name, us in isolated_us.items()},
        # The stage intervals come from HIP events recorded between the
        # layer's launches, so each carries one marker (`marker_us`, an empty
        # bracket timed the same way): they sum above `value`, the plain
        # step; the kernel figures above have the marker taken off, and sum
        # below `value` by the launch gaps of the plain step.
        "marker_us": round(kernel_us["marker"], 2),
        "stage_sum_us": round(sum(in_layer[name] for name in STAGES[1:]), 2),
        "kernel_sum_us": round(sum(kernel_us[name] for name in STAGES[1:]), 2),
        "stage_note": "kernel us = in-layer stage interval less one event marker",
    }
    dominant = max(("logits", "topk", "sparse_mla"), key=lambda k: kernel_us[k])
    traffic = None
    traffic_file = ROOT / "profiles" / "traffic.json"
    if traffic_file.exists():
        traffic = json.loads(traffic_file.read_text()).get(dominant)
    if dominant == "logits":
        achieved = logits_flop / kernel_us["logits"] / 1e6
        roofline = {"kernel": "dsa_indexer_logits_fp8", "bound": "mfma", "achieved": achieved,
                    "peak": PEAKS["fp8_TFLOPs"], "unit": "TFLOP/s"}
    elif dominant == "sparse_mla":
        achieved = mla_flop / kernel_us["sparse_mla"] / 1e6
        roofline = {"kernel": "dsa_sparse_mla_fp8_paged", "bound": "mfma", "achieved": achieved,
                    "peak": PEAKS["bf16_TFLOPs"], "unit": "TFLOP/s"}
    else:
        achieved = topk_bytes / kernel_us["topk"] / 1e3
        roofline = {"kernel": "dsa_indexer_emit_topk", "bound": "hbm", "achieved": achieved,
                    "peak": PEAKS["hbm_GBps"], "unit": "GB/s"}
    roofline["achieved"] = round(roofline["achieved"], 1)
    roofline["frac"] = round(achieved / roofline["peak"], 4)
    roofline["traffic"] = traffic

    result = {
        "metric": "DSA layer us @64K+128 tokens; fp8 logits TFLOPS & sparse-MLA GB/s as % peak",
        "value": round(layer_us, 2),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(layer_us / 1e3, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8 (indexer) + bf16 (sparse MLA)",
        "data": "synthetic (seeded, DeepSeek-V3.2 DSA shapes)",
        "config": {
            "workload": "DSA layer, BASELINE configs 1+2: 65536 history + 128 queries, "
                        "64x128 fp8 indexer, top-2048, 128-head sparse MLA over 656-B fp8 paged KV",
            "history": history,
            "queries": queries,
            "topk": topk,
            "seed": args.seed,
        },
        "roofline": roofline,
        "kernels": kernels,
        # The same layer from the indexer's GEMM outputs (producer launch in
        # place of the prologue); not the headline value.
        "layer_from_gemm_outputs_us": round(projected_layer_us, 2),
    }
    del layer, scores
    torch.cuda.empty_cache()
    if not args.no_config4:
        # BASELINE config 4's layer (131072 + 512, fp8 paged KV), measured the
        # same way; the full config-4 report is `bench.py --config 4`.
        result["config4_fp8_paged_us"] = config4_layer(torch, args, ("fp8_paged",))[
            "formats"]["fp8_paged"]["layer_us"]
    if not args.no_config3:
        # BASELINE config 3 (16 users x 65,536 fp8 history records in pinned host
        # memory, a 262,144-slot pool): one layer for all users, the second of two
        # rounds with the users in sequence and with the overlapped multi-user
        # step; the full report is `bench.py --config 3`.
        rounds, _ = config3_rounds(args, ("sequential", "sequential", "overlapped", "overlapped"))
        result["config3_layer_us"] = {
            "users": args.users,
            "sequential": rounds[1]["layer_us"],
            "overlapped": rounds[3]["layer_us"],
            "fetch_bytes_per_layer": rounds[3]["fetch_bytes_per_layer"],
        }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(inputs, args.cpu_rows, topk)
    print(json.dumps(result))


def stage_times(torch, fns, steps):
    return {name: round(event_time_us(torch, fn, steps), 2) for name, fn in fns.items()}


def mla_reference_f32(torch, mla_q, kv, ids, rows, scale, value_dim=512):
    """Plain fp32 torch sparse MLA of the given query rows over the original
    bf16 KV records (the values the model meant): softmax over the selected
    records (padding ids skipped), then P @ V. On the GPU, per row."""
    out = []
    kv32 = kv.float()
    for r in rows:
        sel = ids[r].long()
        sel = sel[(sel >= 0) & (sel < kv.shape[0])]
        records = kv32.index_select(0, sel)
        logits = torch.matmul(mla_q[r].float(), records.t().contiguous()) * scale
        p = torch.softmax(logits, dim=-1)
        out.append(torch.matmul(p, records[:, :value_dim].contiguous()))
    return torch.stack(out)


def accuracy(torch, got, want):
    """Cosine, max-abs and relative RMS of got against want (fp32)."""
    g, w = got.float().flatten(), want.float().flatten()
    cos = torch.nn.functional.cosine_similarity(g, w, dim=0).item()
    return {"cosine": round(cos, 7), "max_abs": round((g - w).abs().max().item(), 5),
            "rel_rms": round(((g - w).norm() / w.norm()).item(), 6)}


def config4_layer(torch, args, formats=("fp8_paged", "bf16")):
    """Long-context stress: 131072 history + 512 queries, 10 % heavy
    hitters in 8 spans; the layer per KV format, its in-layer stage times (the launches
    the layer runs) and its outputs at 16 spread query rows against an fp32 attention
    over the original bf16 KV."""
    from cxldsagr_amd.layer import DSALayer
    from cxldsagr_amd.workloads import make_layer_inputs

    device = torch.device("cuda", 0)
    history, queries, topk = 131072, 512, 2048
    tokens = history + queries
    inputs = make_layer_inputs(history, queries, seed=args.seed, heavy_fraction=0.10, spans=8)
    result = {"config": 4, "history": history, "queries": queries, "topk": topk, "formats": {}}
    sample_rows = [round(i * (queries - 1) / 15) for i in range(16)]
    kv_all = inputs.kv.to(device)
    mla_q = inputs.mla_q.to(device)
    outputs, reference = {}, None
    for kv_format in formats:
        layer = DSALayer(tokens, device=device, kv_format=kv_format,
                         page_table=inputs.page_table if kv_format == "fp8_paged" else None)
        layer.write_history(inputs.index_k[:history].to(device), kv_all[:history])
        index_q, weights = inputs.index_q.to(device), inputs.weights.to(device)
        index_k_new = inputs.index_k[history:].to(device).contiguous()
        kv_new = kv_all[history:].contiguous()

        def step():
            layer.written = history
            return layer.forward(index_q, index_k_new, weights, mla_q, kv_new)

        out, selection = step()
        spin_up(torch, step)
        for _ in range(args.warmup):
            step()
        layer_us = event_time_us(torch, step, args.steps)
        times, candidates, spilled = in_layer_stage_us(
            torch, layer, history, tokens, topk, args.steps,
            (index_q, index_k_new, weights, mla_q, kv_new))
        pairs = queries * history + queries * (queries + 1) // 2
        logits_flop = 2 * 64 * 128 * pairs
        mla_flop = 2 * queries * topk * 128 * (576 + 512)
        record = 656 if kv_format == "fp8_paged" else 1152
        ids = selection.token_ids
        # Kernel estimates: each stage interval less one event marker.
        kernel = {name: times[name] - times["marker"] for name in STAGES[1:]}
        if reference is None:
            reference = mla_reference_f32(torch, mla_q, kv_all, ids, sample_rows, layer.scale)
        outputs[kv_format] = (out[sample_rows].float(), ids)
        result["formats"][kv_format] = {
            "layer_us": round(layer_us, 2),
            "kernel_us": {name: round(us, 2) for name, us in kernel.items()},
            "stage_us": {name: round(us, 2) for name, us in times.items()},
            "stage_note": "kernel us = in-layer stage interval less one event marker (stage 'marker')",
            "candidates": candidates,
            "spilled_splits": spilled,
            "logits_frac_fp8_peak": round(logits_flop / kernel["logits"] / 1e6 / PEAKS["fp8_TFLOPs"], 4),
            "mla_frac_bf16_peak": round(mla_flop / kernel["sparse_mla"] / 1e6 / PEAKS["bf16_TFLOPs"], 4),
            "gather_GBps": round(queries * topk * record / kernel["sparse_mla"] / 1e3, 1),
            "vs_fp32_over_bf16_kv": accuracy(torch, out[sample_rows], reference),
        }
        del layer, out
        torch.cuda.empty_cache()
    if len(outputs) == 2:
        (a, ids_a), (b, ids_b) = outputs["fp8_paged"], outputs["bf16"]
        result["fp8_vs_bf16"] = accuracy(torch, a, b)
        result["fp8_vs_bf16"]["same_selection"] = bool(torch.equal(ids_a, ids_b))
    result["accuracy_rows"] = sample_rows
    return result


def bench_config4(args):
    import torch

    print(json.dumps(config4_layer(torch, args)))


def pcie_reference(pool, records=262144, reps=5, seed=11):
    """Host-to-device rates on this box for the config-3 recall to be judged by:
    the pinned contiguous hipMemcpyAsync peak (the SDMA engines), the zero-copy
    record gather of the recall (csrc/gather.hip) on random and on address-
    sorted host rows, and a staged alternative (CPU gather of the rows into a
    pinned staging buffer, one hipMemcpyAsync, a device scatter into the slots)
    timed end to end. Same record count and row size (656 B) throughout."""
    import torch

    from cxldsagr_amd import kv_transfer

    device = pool.device
    host = pool.host
    rows = min(records, host.shape[0], pool.slots)
    nbytes = rows * host.shape[1]
    gen = torch.Generator().manual_seed(seed)
    host_ids_cpu = torch.randperm(host.shape[0], generator=gen)[:rows]
    device_ids_cpu = torch.randperm(rows, generator=gen)
    dst = torch.empty((rows, host.shape[1]), dtype=torch.uint8, device=device)
    host_ids = host_ids_cpu.to(device)
    device_ids = device_ids_cpu.to(device)
    sorted_ids = torch.sort(host_ids).values
    staging = torch.empty((rows, host.shape[1]), dtype=torch.uint8, pin_memory=True)
    dstage = torch.empty_like(dst)

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn()
        torch.cuda.synchronize()
        return nbytes * reps / (time.perf_counter() - t0) / 1e9

    def staged():
        torch.index_select(host, 0, host_ids_cpu, out=staging)
        kv_transfer.copy_host_records_async(staging, dstage, host_start=0, device_start=0, count=rows)
        dst.index_copy_(0, device_ids, dstage)

    result = {
        "records": rows,
        "bytes": nbytes,
        "memcpy_h2d_GBps": timed(lambda: kv_transfer.copy_host_records_async(
            host, dst, host_start=0, device_start=0, count=rows)),
        "zero_copy_gather_random_GBps": timed(lambda: kv_transfer.gather_host_records(
            host, dst, host_ids, device_ids)),
        "zero_copy_gather_sorted_GBps": timed(lambda: kv_transfer.gather_host_records(
            host, dst, sorted_ids, device_ids)),
        "staged_cpu_gather_sdma_GBps": timed(staged),
        "cpu_threads": torch.get_num_threads(),
    }
    if kv_transfer.transfer_status(device):
        raise RuntimeError("reference gather flagged an invalid id")
    return {k: round(v, 2) if isinstance(v, float) else v for k, v in result.items()}


def bench_config3(args):
    """The full config-3 report: every round mode, the PCIe reference and the
    serving runner (``config3_rounds`` for the rounds)."""
    rounds, reference = config3_rounds(
        args, ("sequential", "sequential", "overlapped", "overlapped",
               "chunked-2", "chunked-2", "chunked-4", "chunked-4"), reference=True)
    history, queries, topk = 65536, 128, 2048
    print(json.dumps({"config": 3, "users": args.users, "history": history, "queries": queries,
                      "pool_slots": args.users * history // 4, "rounds": rounds,
                      "pcie_reference": reference,
                      "serving": bench_serving(args, args.users, history, queries, topk)}))


def config3_rounds(args, modes, reference=False):
    """GR multi-user recall: `users` sessions of 65536 fp8 history records
    in a pinned host arena, a shared HBM pool of 25 % of all history (262,144 slots for 16
    users), resident indexer keys for every user, rounds of 128 fresh candidate tokens per
    user. Per user and layer: logits -> top-k -> exact recall (gather of the misses from pinned
    host) -> sparse MLA over the pool. One round per entry of ``modes``: "sequential" runs the
    users one after another, as the reference's runner does; "overlapped" runs them through
    ``MultiUserStep`` (each user's recall on a second stream, overlapping its neighbours'
    indexer and sparse MLA); "chunked-N" runs the users one after another, each user's batch
    through ``ChunkedForward`` in N chunks of rows (each chunk's recall overlapping the next
    chunk's indexer and the previous chunk's sparse MLA, within the one request). Returns the
    rounds' reports and, with ``reference``, the box's PCIe reference rates."""
    import torch

    from cxldsagr_amd.layer import OffloadDSALayer
    from cxldsagr_amd.multi_user import ChunkedForward, MultiUserStep
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    device = torch.device("cuda", 0)
    users, history, queries, topk = args.users, 65536, 128, 2048
    tokens = history + queries
    slots = users * history // 4
    pool = TokenPool(users * history, slots, device=device, candidate_slots=2 * queries,
                     history_capacity=history)
    layers = []
    for u in range(users):
        inputs = make_layer_inputs(history, queries, seed=args.seed + u)
        layer = OffloadDSALayer(pool, pool.allocate_session(history), tokens, topk=topk)
        layer.write_history(inputs.index_k[:history].to(device), inputs.kv[:history].to(device))
        layers.append(layer)
        del inputs
    torch.cuda.synchronize()
    step = MultiUserStep(layers)
    chunked = {c: ChunkedForward(pool, c) for c in (2, 4)}

    def round_inputs(round_seed):
        per_user = []
        for u in range(users):
            # Fresh candidates: new queries, index keys and KV for the 128 new tokens.
            fresh = make_layer_inputs(0, queries, seed=round_seed * 1000 + u)
            per_user.append(tuple(getattr(fresh, k).to(device) for k in
                                  ("index_q", "index_k", "weights", "mla_q", "kv")))
        return per_user

    def sequential(batches, timing):
        for layer, (index_q, index_k, weights, mla_q, kv) in zip(layers, batches):
            ids = layer.select(index_q, index_k, weights)
            pool.write_candidates(kv)
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            physical = pool.ensure(ids, layer.session, written=tokens, transient_start=history)
            e1.record()
            timing.append((e0, e1))
            pool.attend(mla_q, physical, layer.scale)

    def chunked_round(batches, chunks):
        for layer, batch in zip(layers, batches):
            if not chunked[chunks].overlaps(layer, queries, transient=True):
                raise RuntimeError("config 3's pool must hold two users' selections")
            chunked[chunks].forward(layer, *batch, transient=True)

    rounds = []
    for r, mode in enumerate(modes):
        batches = round_inputs(r + 1)
        before = pool.metrics()["recalled_records"]
        timing = []
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        if mode == "sequential":
            sequential(batches, timing)
        elif mode == "overlapped":
            step.transient_round(batches)
        else:
            chunked_round(batches, int(mode.split("-")[1]))
        stop.record()
        torch.cuda.synchronize()
        pool.check_status()
        recalled = pool.metrics()["recalled_records"] - before
        fetch_bytes = recalled * 656
        entry = {
            "round": r + 1,
            "mode": mode,
            "layer_us": round(start.elapsed_time(stop) * 1e3, 1),
            "fetch_records": recalled,
            "fetch_bytes_per_layer": fetch_bytes,
            "fetch_bytes_per_user": fetch_bytes // users,
        }
        if timing:
            fetch_us = sum(a.elapsed_time(b) for a, b in timing) * 1e3
            entry["recall_us"] = round(fetch_us, 1)
            entry["pcie_GBps"] = round(fetch_bytes / fetch_us / 1e3, 2) if fetch_us > 0 else None
        else:
            entry["pcie_GBps_over_layer"] = round(fetch_bytes / (entry["layer_us"] * 1e3), 2)
        rounds.append(entry)
    pcie = pcie_reference(pool) if reference else None
    del step, chunked, layers, pool
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rounds, pcie


def bench_serving(args, users, history, queries, topk):
    """The GR serving runner (``cxldsagr_amd.serving``) on config 3's users: a
    host arena for three quarters of them, so that the LRU evicts; two passes
    over the users (the second revisits). Per request: admission, history
    prefill on a miss (index K into the resident cache, fp8 records written
    straight into pinned host pages), the transient candidate step with its
    exact recall. Reports per-pass request latencies, hits and fetched bytes
    (the second pass visits the users in reverse order)."""
    import torch

    from cxldsagr_amd.serving import GRServingRunner
    from cxldsagr_amd.token_pool import TokenPool
    from cxldsagr_amd.workloads import make_layer_inputs

    device = torch.device("cuda", 0)
    cached = max(1, users * 3 // 4)
    pool = TokenPool(cached * history, users * history // 4, device=device,
                     candidate_slots=queries, history_capacity=history)

    # Each user's projected history, generated once on the device (outside
    # the timed requests; a miss then writes it into the caches).
    histories = []
    for u in range(users):
        x = make_layer_inputs(history, queries, seed=args.seed + u)
        histories.append([(x.index_k[:history].to(device), x.kv[:history].to(device))])
        del x

    def history_of(u):
        return lambda: histories[u]

    passes = []
    with GRServingRunner([pool], topk=topk) as runner:
        for p in range(2):
            metrics = []
            # The second pass visits the users in reverse order, so the most
            # recent ones hit before the evicted ones come back.
            for u in (range(users) if p == 0 else reversed(range(users))):
                fresh = make_layer_inputs(0, queries, seed=(p + 10) * 1000 + u)
                batch = [tuple(getattr(fresh, k).to(device) for k in
                               ("index_q", "index_k", "weights", "mla_q", "kv"))]
                result = runner.execute({"user_id": u, "signature": ("history", u),
                                         "history_tokens": history, "history": history_of(u),
                                         "candidates": batch})
                metrics.append(result.metrics)
            hits = [m for m in metrics if m["prefix_cache_hit"]]
            passes.append({
                "pass": p + 1,
                "requests": len(metrics),
                "hits": len(hits),
                "evictions": sum(len(m["evicted_users"]) for m in metrics),
                "latency_ms_mean": round(sum(m["latency_ms"] for m in metrics) / len(metrics), 2),
                "prefix_ms_mean_on_miss": round(
                    sum(m["prefix_ms"] for m in metrics if not m["prefix_cache_hit"])
                    / max(1, len(metrics) - len(hits)), 2),
                "extend_ms_mean": round(sum(m["extend_ms"] for m in metrics) / len(metrics), 2),
                "fetch_bytes": sum(m["fetch_bytes"] for m in metrics),
            })
    return {"arena_users": cached, "pool_slots": users * history // 4, "passes": passes}


if __name__ == "__main__":
    main()
