"""Indexer input producers on MI355X: the indexer half of the projection step.

The reference's ``CheckpointAttention.project``
(``models/deepseek_v32/projections.py:182-257``) produces the indexer inputs
of a layer from the normalised hidden states ``x`` and the query LoRA
activations ``qr``:

* ``index_q = index_wq(qr)`` viewed ``[T, 64, 128]`` and
  ``index_k = LayerNorm(index_wk(x).float()).bfloat16()`` (``:114-121``);
* non-interleaved RoPE on the first 64 dims of both
  (``apply_rope_pair(..., interleaved=False)``, ``:236-238``;
  ``rotary.py:47-85``);
* ``quantize_index`` of both (``:239-240``);
* ``weights = (weights_proj(x.float()) * 64**-0.5) * q_scale * 128**-0.5``
  (``:241-242``);

and the runner writes index K into the layer's resident cache
(``models/deepseek_v32/attention.py:323-326``).

Here the three projections are plain library GEMMs (``torch.nn.functional.
linear`` on the device, hipBLASLt); everything after them - LayerNorm, both
RoPEs, both quantisations, the weight scaling and fold, the index-cache
write and, optionally, the new tokens' fp8 KV records - is one gfx950 launch
(``dsa_index_producer_fp8`` in ``csrc/quantize.hip``), enqueued on the
current stream without host synchronisation.
"""

import math
from dataclasses import dataclass

import torch

from cxldsagr_amd import _native
from cxldsagr_amd.attention import PAGE_TOKENS, QK_DIM, RECORD_BYTES

INDEX_HEADS = 64
INDEX_DIM = 128
ROPE_DIM = 64


def rotary_frequencies(rope_dim=64, rope_theta=10000.0, max_seq_len=163840,
                       original_seq_len=4096, beta_fast=32.0, beta_slow=1.0, rope_factor=40.0):
    """YaRN-corrected RoPE frequencies, float32 ``[rope_dim // 2]`` on the CPU.

    The arithmetic of ``rotary_frequencies`` (``models/deepseek_v32/rotary.py:26-44``)
    with the DeepSeek-V3.2 defaults (``config.py:18,26-31``): the base
    ``theta**(-2i/d)``, blended towards ``freq / rope_factor`` over the dims
    between the beta_fast and beta_slow correction dims when the context
    exceeds the original one.
    """
    dim = rope_dim
    freq = rope_theta ** (-torch.arange(0, dim, 2).float() / dim)
    if max_seq_len > original_seq_len:
        def correction(rotations):
            return (dim * math.log(original_seq_len / (rotations * 2 * math.pi))
                    / (2 * math.log(rope_theta)))

        low = max(math.floor(correction(beta_fast)), 0)
        high = min(math.ceil(correction(beta_slow)), dim - 1)
        if low == high:
            high += 0.001
        ramp = ((torch.arange(dim // 2).float() - low) / (high - low)).clamp(0, 1)
        freq = freq * (1 - ramp) + freq / rope_factor * ramp
    return freq


def rotary_table(positions, frequencies):
    """Per-call RoPE table ``cat(cos, sin)`` f32 ``[T, 64]`` for fp32 positions.

    The table ``prepare_rotary_cache`` builds (``rotary.py:59-64``) from
    ``angles = positions[:, None] * frequencies[None, :]``
    (``projections.py:211``); token ``t`` reads row ``t``.
    """
    if positions.dtype != torch.float32 or positions.ndim != 1:
        raise ValueError("positions must be one FP32 value per token")
    angles = positions[:, None] * frequencies.to(positions.device)[None, :]
    return torch.cat((angles.cos(), angles.sin()), dim=-1).contiguous()


def index_producer(q_proj, k_proj, head_logits, norm_weight, norm_bias, eps, cos_sin,
                   rope_rows=None, *, index_keys=None, index_scales=None, q_fold=False,
                   kv=None, kv_cache=None, page_table=None, token_offset=0, status=None,
                   head_scales=(INDEX_HEADS ** -0.5, INDEX_DIM ** -0.5), floors=None,
                   key_cache=None, key_cache_scales=None, topk=2048):
    """Index Q/K from their GEMM outputs, in one launch.

    ``q_proj`` bf16 ``[T, 64, 128]`` (``index_wq(qr)``), ``k_proj`` bf16
    ``[T, 128]`` (``index_wk(x)``), ``head_logits`` f32 ``[T, 64]``
    (``weights_proj(x.float())``), LayerNorm ``norm_weight``/``norm_bias``
    f32 ``[128]`` and ``eps``, ``cos_sin`` f32 ``[P, 64]`` (``rotary_table``)
    and optional ``rope_rows`` int32 ``[T]`` (row of each token; default
    ``t``). Index K goes to ``index_keys``/``index_scales`` when given (the
    resident cache rows of these tokens), else to new tensors. With ``kv``
    (bf16 ``[T, 576]``) the tokens' fp8 records are also packed into
    ``kv_cache`` behind ``page_table`` at ``token_offset``. With ``floors``
    (int32 ``[T, 2]``) the same launch writes the candidate top-k's per-row
    floors (``indexer.select_topk``) for queries at positions
    ``token_offset ..`` over the resident index cache ``key_cache`` fp8
    ``[>= token_offset, 128]`` / ``key_cache_scales`` f32, sampled from its
    first ``token_offset`` rows.

    Returns ``(index_q fp8 [T,64,128], q_scale f32 [T,64,1], weights f32
    [T,64], index_k fp8 [T,128], k_scale f32 [T], q_fold f32 [T,4,128] or
    None)``; ``weights`` is the reference's ``index_weights`` with the q-scale
    folded in.
    """
    tokens = q_proj.shape[0] if isinstance(q_proj, torch.Tensor) and q_proj.ndim else 0
    device = q_proj.device
    _native.require_gfx950(device, "index producers")
    checks = (
        (q_proj, (tokens, INDEX_HEADS, INDEX_DIM), torch.bfloat16, "q_proj"),
        (k_proj, (tokens, INDEX_DIM), torch.bfloat16, "k_proj"),
        (head_logits, (tokens, INDEX_HEADS), torch.float32, "head_logits"),
        (norm_weight, (INDEX_DIM,), torch.float32, "norm_weight"),
        (norm_bias, (INDEX_DIM,), torch.float32, "norm_bias"),
    )
    for tensor, shape, dtype, name in checks:
        if (not isinstance(tensor, torch.Tensor) or tuple(tensor.shape) != shape
                or tensor.dtype != dtype or tensor.device != device):
            raise ValueError(f"{name} must be {dtype} {shape} on {device}")
    if (not isinstance(cos_sin, torch.Tensor) or cos_sin.ndim != 2 or cos_sin.shape[1] != ROPE_DIM
            or cos_sin.dtype != torch.float32 or cos_sin.device != device):
        raise ValueError(f"cos_sin must be FP32 [rows, {ROPE_DIM}] on {device}")
    if rope_rows is None:
        if cos_sin.shape[0] < tokens:
            raise ValueError("cos_sin needs a row per token when rope_rows is not given")
    elif (rope_rows.dtype != torch.int32 or tuple(rope_rows.shape) != (tokens,)
          or rope_rows.device != device):
        raise ValueError("rope_rows must be int32 [tokens] on the producer device")
    if not math.isfinite(eps) or eps < 0:
        raise ValueError("eps must be finite and nonnegative")
    q_proj, k_proj, head_logits, norm_weight, norm_bias, cos_sin = (
        _aligned(t.contiguous()) for t in (q_proj, k_proj, head_logits, norm_weight, norm_bias,
                                           cos_sin))
    if rope_rows is not None:
        rope_rows = rope_rows.contiguous()

    q8 = torch.empty(q_proj.shape, dtype=torch.float8_e4m3fn, device=device)
    q_scales = torch.empty((tokens, INDEX_HEADS, 1), dtype=torch.float32, device=device)
    weights = torch.empty((tokens, INDEX_HEADS), dtype=torch.float32, device=device)
    fold = torch.empty((tokens, 4, INDEX_DIM), dtype=torch.float32, device=device) if q_fold else None
    if index_keys is None:
        index_keys = torch.empty((tokens, INDEX_DIM), dtype=torch.float8_e4m3fn, device=device)
        index_scales = torch.empty(tokens, dtype=torch.float32, device=device)
    elif (index_keys.dtype != torch.float8_e4m3fn or tuple(index_keys.shape) != (tokens, INDEX_DIM)
          or not index_keys.is_contiguous() or index_scales is None
          or index_scales.dtype != torch.float32 or tuple(index_scales.shape) != (tokens,)
          or not index_scales.is_contiguous()
          or index_keys.device != device or index_scales.device != device):
        raise ValueError("index_keys/index_scales must be contiguous fp8 [T,128] / FP32 [T] rows")
    pages = 0
    if kv is not None:
        if (kv.dtype != torch.bfloat16 or tuple(kv.shape) != (tokens, QK_DIM)
                or kv.device != device):
            raise ValueError(f"kv must be BF16 ({tokens}, {QK_DIM}) on {device}")
        if (kv_cache is None or kv_cache.dtype != torch.uint8 or kv_cache.ndim != 3
                or tuple(kv_cache.shape[1:]) != (PAGE_TOKENS, RECORD_BYTES)
                or not kv_cache.is_contiguous() or kv_cache.device != device
                or page_table is None or page_table.dtype != torch.int32
                or page_table.device != device or not page_table.is_contiguous()):
            raise ValueError("kv needs a contiguous uint8 [pages, 64, 656] cache and an int32 "
                             "page table")
        if page_table.numel() * PAGE_TOKENS < token_offset + tokens:
            raise ValueError("page_table does not cover the appended tokens")
        kv = _aligned(kv.contiguous())
        pages = kv_cache.shape[0]
    floor_args = ()
    if floors is not None:
        if (floors.dtype != torch.int32 or tuple(floors.shape) != (tokens, 2)
                or not floors.is_contiguous() or floors.device != device):
            raise ValueError("floors must be contiguous int32 [tokens, 2]")
        if (key_cache is None or key_cache.dtype != torch.float8_e4m3fn or key_cache.ndim != 2
                or key_cache.shape[1] != INDEX_DIM or key_cache.shape[0] < token_offset
                or not key_cache.is_contiguous() or key_cache.device != device
                or key_cache_scales is None or key_cache_scales.dtype != torch.float32
                or key_cache_scales.shape[0] < token_offset or key_cache_scales.device != device):
            raise ValueError("floors need the resident index cache: fp8 [>= token_offset, 128] "
                             "keys and FP32 scales")
        if type(topk) is not int or not 1 <= topk <= 2048:
            raise ValueError("topk must be an integer in [1, 2048]")
        floor_args = (_native.ptr(key_cache), _native.ptr(key_cache_scales), int(token_offset),
                      topk, _native.ptr(floors))
    if tokens == 0:
        return q8, q_scales, weights, index_keys, index_scales, fold
    pre, post = head_scales
    with torch.cuda.device(device):
        _native.call(
            "dsa_index_producer_floors_fp8" if floor_args else "dsa_index_producer_fp8",
            _native.ptr(q_proj), tokens, _native.ptr(head_logits), float(pre), float(post),
            _native.ptr(k_proj), _native.ptr(norm_weight), _native.ptr(norm_bias), float(eps),
            _native.ptr(cos_sin), cos_sin.shape[0], _native.ptr(rope_rows),
            _native.ptr(q8), _native.ptr(q_scales), _native.ptr(weights), _native.ptr(fold),
            _native.ptr(index_keys), _native.ptr(index_scales),
            _native.ptr(kv), int(token_offset), _native.ptr(page_table), pages,
            _native.ptr(kv_cache if kv is not None else None), _native.ptr(status),
            *floor_args, _native.stream_of(device),
        )
    return q8, q_scales, weights, index_keys, index_scales, fold


def _aligned(t):
    """A 16-byte-aligned copy when the storage offset breaks alignment."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


@dataclass
class IndexProjected:
    """GEMM outputs of one token batch, before the producer launch."""

    q_proj: torch.Tensor       # bf16 [T, 64, 128]
    k_proj: torch.Tensor       # bf16 [T, 128]
    head_logits: torch.Tensor  # f32 [T, 64]
    cos_sin: torch.Tensor      # f32 [T, 64]


class IndexerProjection:
    """The indexer's projection weights of one layer.

    ``index_wq`` bf16 ``[64*128, q_lora_rank]``, ``index_wk`` bf16
    ``[128, dim]``, ``weights_proj`` f32 ``[64, dim]``, LayerNorm
    ``norm_weight``/``norm_bias`` f32 ``[128]`` (the checkpoint tensors
    ``indexer.wq_b``, ``indexer.wk``, ``indexer.weights_proj``,
    ``indexer.k_norm.{weight,bias}``, ``projections.py:85-96``), and the
    RoPE ``frequencies`` f32 ``[32]``.
    """

    def __init__(self, index_wq, index_wk, weights_proj, norm_weight, norm_bias, frequencies,
                 *, eps=1e-6):
        if index_wq.ndim != 2 or index_wq.shape[0] != INDEX_HEADS * INDEX_DIM:
            raise ValueError("index_wq must be [64 * 128, q_lora_rank]")
        if index_wk.ndim != 2 or index_wk.shape[0] != INDEX_DIM:
            raise ValueError("index_wk must be [128, dim]")
        if tuple(weights_proj.shape) != (INDEX_HEADS, index_wk.shape[1]):
            raise ValueError("weights_proj must be [64, dim]")
        if tuple(frequencies.shape) != (ROPE_DIM // 2,):
            raise ValueError("frequencies must hold 32 values")
        self.index_wq = index_wq.to(torch.bfloat16).contiguous()
        self.index_wk = index_wk.to(torch.bfloat16).contiguous()
        self.weights_proj = weights_proj.to(torch.float32).contiguous()
        self.norm_weight = norm_weight.to(torch.float32).contiguous()
        self.norm_bias = norm_bias.to(torch.float32).contiguous()
        self.frequencies = frequencies.to(device=self.index_wq.device, dtype=torch.float32)
        self.eps = float(eps)
        self.device = self.index_wq.device

    def project(self, x, qr, positions):
        """The three GEMMs and the RoPE table (library calls; no producer yet)."""
        if x.ndim != 2 or qr.ndim != 2 or len(x) != len(qr) or x.dtype != torch.bfloat16:
            raise ValueError("x [T, dim] and qr [T, q_lora_rank] must be BF16 with equal T")
        tokens = len(x)
        q_proj = torch.nn.functional.linear(qr, self.index_wq).view(tokens, INDEX_HEADS, INDEX_DIM)
        k_proj = torch.nn.functional.linear(x, self.index_wk)
        head_logits = torch.nn.functional.linear(x.float(), self.weights_proj)
        return IndexProjected(q_proj, k_proj, head_logits, rotary_table(positions, self.frequencies))

    def produce(self, projected, **kwargs):
        """``index_producer`` over ``projected`` with this layer's norm parameters."""
        return index_producer(projected.q_proj, projected.k_proj, projected.head_logits,
                              self.norm_weight, self.norm_bias, self.eps, projected.cos_sin,
                              **kwargs)
