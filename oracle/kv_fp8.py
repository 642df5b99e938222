"""A8: the 656-byte fp8 paged KV record (TEST INFRASTRUCTURE ONLY).

The reference stores bf16 576-wide records (1152 B/token,
``operators/deepseek_v32/README.md:55``); the fp8 paged format is defined by
this build's benchmark configuration, so there is no reference code to follow.
Layout of one token record:

* bytes ``[0, 512)``: e4m3fn latent, four tiles of 128 values, each tile
  quantised with the A1 rule (UE8M0 scale, ``oracle.quantize``);
* bytes ``[512, 528)``: the four fp32 tile scales, little endian;
* bytes ``[528, 656)``: the 64 RoPE values as raw bf16.

Tokens live in 64-token pages: token ``t`` is row ``page_table[t // 64] * 64 +
t % 64`` of the ``[pages * 64, 656]`` byte array. Dequantisation is
``decode(code) * scale``; with a power-of-two scale this value is exactly a
bf16 value, so attention over the dequantised cache is attention over a bf16
cache.

Pinned by ``tests/test_oracle_kv_fp8.py``: every byte field against torch's
own float8 cast with the reference's log2/ceil UE8M0 scale per tile (codes,
little-endian fp32 scales at bytes 512-527, RoPE bits at 528-655), the
encode/decode round trip within the e4m3 half-ulp bound, exact bf16
representability of every dequantised value, and page-table addressing on a
hand-built two-page permuted table and a random permutation. The same file
plants mistakes in copies of the encoder and requires the pins to catch each.
"""

import numpy as np

from oracle import fp8, quantize

RECORD_BYTES = 656
PAGE_TOKENS = 64
LATENT = 512
ROPE = 64
TILE = 128


def encode_records(latent_rope_bf16_bits):
    """uint16 bf16 bits [T, 576] -> uint8 records [T, 656]."""
    bits = np.asarray(latent_rope_bf16_bits, dtype=np.uint16)
    tokens = bits.shape[0]
    latent = fp8.bf16_bits_to_f32(bits[:, :LATENT]).reshape(tokens, LATENT // TILE, TILE)
    codes, scales = quantize.quantize_index(latent, "ue8m0")
    out = np.zeros((tokens, RECORD_BYTES), dtype=np.uint8)
    out[:, :LATENT] = codes.reshape(tokens, LATENT)
    out[:, LATENT:LATENT + 16] = np.ascontiguousarray(
        scales.reshape(tokens, 4).astype("<f4")).view(np.uint8)
    out[:, LATENT + 16:] = np.ascontiguousarray(
        bits[:, LATENT:].astype("<u2")).view(np.uint8)
    return out


def decode_records(records):
    """uint8 records [T, 656] -> float32 [T, 576] (exact bf16 values)."""
    records = np.ascontiguousarray(records, dtype=np.uint8)
    tokens = records.shape[0]
    codes = records[:, :LATENT].reshape(tokens, 4, TILE)
    scales = np.ascontiguousarray(records[:, LATENT:LATENT + 16]).view("<f4").reshape(tokens, 4, 1)
    latent = (fp8.decode(codes) * scales.astype(np.float32)).reshape(tokens, LATENT)
    rope = fp8.bf16_bits_to_f32(
        np.ascontiguousarray(records[:, LATENT + 16:]).view("<u2").reshape(tokens, ROPE))
    return np.concatenate([latent, rope], axis=1).astype(np.float32)


def physical_rows(page_table, tokens):
    """Physical row of each logical token ``0..tokens-1``."""
    t = np.arange(tokens, dtype=np.int64)
    return np.asarray(page_table, dtype=np.int64)[t // PAGE_TOKENS] * PAGE_TOKENS + t % PAGE_TOKENS


def build_cache(latent_rope_bf16_bits, page_table, pages):
    """Pack tokens into a paged cache ``uint8 [pages, 64, 656]``."""
    records = encode_records(latent_rope_bf16_bits)
    cache = np.zeros((pages * PAGE_TOKENS, RECORD_BYTES), dtype=np.uint8)
    cache[physical_rows(page_table, records.shape[0])] = records
    return cache.reshape(pages, PAGE_TOKENS, RECORD_BYTES)


def logical_records(cache, page_table, tokens):
    """Dequantised float32 [tokens, 576] in logical token order."""
    flat = np.asarray(cache).reshape(-1, RECORD_BYTES)
    return decode_records(flat[physical_rows(page_table, tokens)])
