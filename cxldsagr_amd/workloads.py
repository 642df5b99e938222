"""Seeded synthetic inputs for the benchmark configurations.

Generation rules (seeded ``torch.Generator`` on the CPU, default seed 947 as in
the reference's observation harness,
``experiments/deepseek_v32_observation/src/attention_workload.py:107``):

* indexer ``q [Q,64,128]`` and ``k [N,128]`` bf16 ~ N(0,1);
* heavy hitters: a fraction of key positions (5 % by default, a seeded
  ``randperm``; or ``spans`` contiguous runs for the long-context stress
  case) get ``k[j] += 2 u`` with ``u = m / |m|``, ``m`` the mean of ``q`` over
  rows and heads - one fixed reading of "shifted by +2x the mean query
  direction";
* per-head weights ``[Q,64]`` ~ N(0,1)/8 fp32;
* sparse MLA ``q [Q,128,576]`` and latent KV ``[N,576]`` bf16 ~ N(0,1);
  softmax scale ``576 ** -0.5``;
* the paged KV page table is a seeded ``randperm`` of the pages.

Inputs are produced on the CPU and moved to the device; quantisation and
cache packing then run through the HIP kernels.
"""

from dataclasses import dataclass

import torch

PAGE_TOKENS = 64


@dataclass
class LayerInputs:
    history: int
    queries: int
    index_q: torch.Tensor      # bf16 [Q, 64, 128]
    index_k: torch.Tensor      # bf16 [N, 128]
    weights: torch.Tensor      # f32 [Q, 64]
    mla_q: torch.Tensor        # bf16 [Q, heads, 576]
    kv: torch.Tensor           # bf16 [N, 576]
    page_table: torch.Tensor   # int32 [ceil(N/64)]
    heavy: torch.Tensor        # int64 positions of heavy-hitter keys
    seed: int

    @property
    def tokens(self):
        return self.history + self.queries

    @property
    def pages(self):
        return (self.tokens + PAGE_TOKENS - 1) // PAGE_TOKENS

    def to(self, device):
        for name in ("index_q", "index_k", "weights", "mla_q", "kv", "page_table"):
            setattr(self, name, getattr(self, name).to(device))
        return self


def make_layer_inputs(history, queries, *, seed=947, heads=128, heavy_fraction=0.05,
                      spans=None):
    """Inputs of one DSA layer with ``history`` cached tokens and ``queries`` new ones."""
    if queries < 1:
        # The heavy-hitter direction is the mean query; without queries it is undefined.
        raise ValueError("make_layer_inputs needs at least one query token")
    gen = torch.Generator().manual_seed(seed)
    tokens = history + queries
    index_q = torch.randn(queries, 64, 128, generator=gen).bfloat16()
    index_k = torch.randn(tokens, 128, generator=gen)
    weights = torch.randn(queries, 64, generator=gen) / 8
    mean = index_q.float().mean(dim=(0, 1))
    direction = mean / mean.norm()
    count = int(round(heavy_fraction * tokens))
    if spans is None:
        heavy = torch.randperm(tokens, generator=gen)[:count]
    else:
        starts = torch.randperm(max(1, tokens - count // spans), generator=gen)[:spans]
        length = count // spans
        heavy = torch.unique(torch.cat([torch.arange(s, s + length) for s in starts.tolist()]))
        heavy = heavy[heavy < tokens]
    index_k[heavy] += 2 * direction
    mla_q = torch.randn(queries, heads, 576, generator=gen).bfloat16()
    kv = torch.randn(tokens, 576, generator=gen).bfloat16()
    pages = (tokens + PAGE_TOKENS - 1) // PAGE_TOKENS
    page_table = torch.randperm(pages, generator=gen).to(torch.int32)
    return LayerInputs(history, queries, index_q, index_k.bfloat16(), weights, mla_q, kv,
                       page_table, heavy.long(), seed)


CONFIGS = {
    # name: (history, queries, kwargs)
    "config0": (4096, 128, {}),
    "config1_2": (65536, 128, {}),
    "config4": (131072, 512, {"heavy_fraction": 0.10, "spans": 8}),
}
