"""Writes tests/golden/dsa_small.npz: small seeded inputs of every hot-path
stage and the CPU oracle's outputs for them (quantise, logits, top-k, fp8 KV
pack, sparse MLA over the paged cache).

The reference ships no data fixtures for this path (its tests draw inputs
from seeds), so these vectors come from the oracle. They pin nothing by
themselves: each oracle function is pinned independently in
tests/test_oracle_*.py (the reference's own test cases restated, torch's
casts, closed forms and brute force). Committed vectors keep the GPU tests
independent of later oracle edits, and tests/test_golden.py re-derives them
to catch any drift.

Run from the repository root: python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import fp8 as ofp8  # noqa: E402
from oracle import kv_fp8 as okv  # noqa: E402
from oracle import logits as ologits  # noqa: E402
from oracle import quantize as oquant  # noqa: E402
from oracle import sparse_mla as omla  # noqa: E402
from oracle import topk as otopk  # noqa: E402

OUT = Path(__file__).resolve().parent / "dsa_small.npz"
SEED = 521
MLA_SCALE = 576 ** -0.5


def bf16_bits(x):
    return ofp8.f32_to_bf16_bits(np.asarray(x, dtype=np.float32))


def bits_to_f32(bits):
    return ofp8.bf16_bits_to_f32(bits)


def make():
    rng = np.random.default_rng(SEED)
    g = {}
    # A1: rows at several magnitudes, a zero row, a subnormal-scale row, a wide row.
    x = rng.standard_normal((12, 128)).astype(np.float32)
    x *= np.array([1, 1e-3, 1e3, 0.5, 2, 7, 1e-30, 1, 3e4, 1, 1, 1], dtype=np.float32)[:, None]
    x[5] = 0.0
    x[10, ::7] = 448.0
    g["quant_x_bits"] = bf16_bits(x)
    codes, scales = oquant.quantize_index(bits_to_f32(g["quant_x_bits"]))
    g["quant_codes"], g["quant_scales"] = codes, scales

    # A4: 4 query rows at the end of 100 tokens (causal tail), fp8 operands.
    q_codes, q_scales = oquant.quantize_index(bits_to_f32(bf16_bits(rng.standard_normal((4, 64, 128)))))
    k_codes, k_scales = oquant.quantize_index(bits_to_f32(bf16_bits(rng.standard_normal((100, 128)))))
    weights = (rng.standard_normal((4, 64)).astype(np.float32) / 8 * q_scales[..., 0]).astype(np.float32)
    g.update(logits_q=q_codes, logits_k=k_codes, logits_w=weights,
             logits_kscale=k_scales[:, 0].astype(np.float32), logits_query_start=np.int64(96))
    g["logits_out"] = ologits.logits(q_codes, k_codes, weights, g["logits_kscale"], 96)

    # A6: ties (values on a coarse grid), -inf tails, a -0.0 / +0.0 pair, k = 300.
    scores = (np.round(rng.standard_normal((4, 3000)) * 8) / 8).astype(np.float32)
    scores[1, 2500:] = -np.inf
    scores[2, :2] = np.array([-0.0, 0.0], dtype=np.float32)
    scores[3, :] = 0.25
    g["topk_scores"], g["topk_k"] = scores, np.int64(300)
    g["topk_values"], g["topk_ids"] = otopk.exact_topk(scores, 300)

    # A8 + A7: 96 tokens in two pages (permuted), 2 query rows x 64 heads,
    # selections with duplicates, padding and an id past the last token.
    kv_bits = bf16_bits(rng.standard_normal((96, 576)))
    table = np.array([1, 0], dtype=np.int32)
    cache = okv.build_cache(kv_bits, table, 2)
    ids = rng.integers(0, 96, size=(2, 40)).astype(np.int32)
    ids[0, :4] = [7, 7, 7, -1]
    ids[1, -3:] = [96, -5, 95]
    q_bits = bf16_bits(rng.standard_normal((2, 64, 576)))
    records = okv.logical_records(cache, table, 96)
    out_bits, _ = omla.sparse_mla(bits_to_f32(q_bits), records, ids, MLA_SCALE)
    g.update(kv_bits=kv_bits, kv_table=table, kv_cache=cache, mla_q_bits=q_bits, mla_ids=ids,
             mla_scale=np.float32(MLA_SCALE), mla_out_bits=out_bits)
    return g


if __name__ == "__main__":
    np.savez_compressed(OUT, **make())
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
