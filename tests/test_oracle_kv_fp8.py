"""Pins of the oracle's 656-byte fp8 paged KV record (CPU only).

The record has no reference counterpart, so it is pinned by its own closed
forms, each computed by a route that does not reuse ``oracle.kv_fp8``:

* every byte field against torch: latent codes equal torch's own
  ``(x / s).clamp(-448, 448).to(float8_e4m3fn)`` with ``s`` the log2/ceil
  UE8M0 scale of the reference's eager quantiser
  (operators/deepseek_v32/indexer/quantization.py:12-21), per 128-value
  tile; bytes 512-527 are those four scales as little-endian fp32; bytes
  528-655 are the RoPE bf16 bits unchanged;
* the round trip: every dequantised latent value lies within half an e4m3
  unit in the last place (times the tile scale) of its input, and is an
  exact bf16 value;
* page addressing on a hand-built two-page permuted table, and on a
  random permutation against a scalar loop.

``test_pins_reject_planted_mistakes`` plants mistakes in copies of the
encoder (two bytes of a scale swapped, two tile scales swapped, tiles of 64
instead of 128, the RoPE half byte-swapped, one scale for the whole record)
and requires each to fail.
"""

import numpy as np
import pytest
import torch

from oracle import fp8
from oracle import kv_fp8 as okv


def _bf16_bits(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).bfloat16().view(
        torch.int16).numpy().view(np.uint16)


def _inputs(tokens, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((tokens, 576)).astype(np.float32)
    x[:, :512] *= np.exp2(rng.integers(-12, 8, (tokens, 4))).repeat(128, axis=1).astype(np.float32)
    x[0, :128] = 0.0                 # an all-zero tile: scale from the 1e-4 floor
    x[1, 200] = 1000.0               # one tile with a large outlier
    return _bf16_bits(x)


def _torch_tile(values_f32):
    """Codes and scale of one 128-value tile, torch's log2/ceil formulation."""
    t = torch.from_numpy(values_f32.astype(np.float32))
    amax = t.abs().amax().clamp_min(1e-4)
    scale = torch.exp2(torch.ceil(torch.log2(amax / 448.0)))
    codes = (t / scale).clamp(-448, 448).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    return codes, np.float32(scale.item())


# ----------------------------------------------------------------- the checks
def check_fields_against_torch(encode, bits):
    records = encode(bits)
    assert records.shape == (bits.shape[0], 656) and records.dtype == np.uint8
    values = fp8.bf16_bits_to_f32(bits)
    for t in range(bits.shape[0]):
        for tile in range(4):
            codes, scale = _torch_tile(values[t, 128 * tile:128 * tile + 128])
            np.testing.assert_array_equal(records[t, 128 * tile:128 * tile + 128], codes)
            stored = records[t, 512 + 4 * tile:516 + 4 * tile].tobytes()
            assert stored == np.float32(scale).astype("<f4").tobytes(), (t, tile)
        assert records[t, 528:].tobytes() == bits[t, 512:].astype("<u2").tobytes()


def check_round_trip(encode, bits):
    records = encode(bits)
    values = fp8.bf16_bits_to_f32(bits).astype(np.float64)
    decoded = okv.decode_records(records).astype(np.float64)
    scales = np.frombuffer(records[:, 512:528].tobytes(), "<f4").reshape(-1, 4).astype(np.float64)
    s = np.repeat(scales, 128, axis=1)
    y = np.abs(values[:, :512]) / s
    # e4m3 unit in the last place of |y|: 2^(e - 3) for 2^e <= |y| < 2^(e+1)
    # in the normal range, 2^-9 below 2^-6.
    e = np.floor(np.log2(np.maximum(y, 2.0**-6)))
    ulp = np.exp2(e - 3)
    assert (np.abs(decoded[:, :512] - values[:, :512]) <= 0.5 * ulp * s).all()
    assert np.array_equal(decoded[:, 512:], values[:, 512:])
    # Every dequantised value is exactly a bf16 value.
    f32 = decoded.astype(np.float32)
    assert np.array_equal(fp8.bf16_bits_to_f32(_bf16_bits(f32)), f32)


CHECKS = [check_fields_against_torch, check_round_trip]


@pytest.mark.parametrize("seed", [0, 1])
@pytest.mark.parametrize("check", range(len(CHECKS)))
def test_oracle_passes_pin(check, seed):
    CHECKS[check](okv.encode_records, _inputs(40, seed))


def test_two_page_permuted_table_by_hand():
    """Tokens 0..99 over logical pages [0, 1] mapped to physical pages [1, 0]
    of a two-page cache: token t < 64 lands in physical row 64 + t, token
    t >= 64 in row t - 64."""
    bits = _inputs(100, 3)
    cache = okv.build_cache(bits, np.array([1, 0]), 2).reshape(-1, 656)
    records = okv.encode_records(bits)
    for t in range(100):
        row = 64 + t if t < 64 else t - 64
        np.testing.assert_array_equal(cache[row], records[t])
    # Rows no token maps to stay zero.
    assert not cache[36:64].any()
    np.testing.assert_array_equal(okv.logical_records(cache, np.array([1, 0]), 100),
                                  okv.decode_records(records))


def test_random_page_table_against_scalar_loop():
    rng = np.random.default_rng(7)
    pages, tokens = 9, 500
    table = rng.permutation(pages)
    bits = _inputs(tokens, 4)
    cache = okv.build_cache(bits, table, pages).reshape(-1, 656)
    records = okv.encode_records(bits)
    for t in range(tokens):
        page, slot = divmod(t, 64)
        np.testing.assert_array_equal(cache[int(table[page]) * 64 + slot], records[t])


def test_zero_tile_scale_is_the_floor():
    bits = _inputs(2, 0)
    records = okv.encode_records(bits)
    scale = np.frombuffer(records[0, 512:516].tobytes(), "<f4")[0]
    # 1e-4 / 448 rounded up to a power of two.
    assert scale == np.float32(2.0**-22) and not records[0, :128].any()


# ------------------------------------------------------------ planted mistakes
def _mutant(kind):
    def encode(bits):
        out = okv.encode_records(bits)
        if kind == "swapped_scale_bytes":
            out[:, [514, 515]] = out[:, [515, 514]]
        elif kind == "swapped_tile_scales":
            out[:, 512:520] = np.concatenate([out[:, 516:520], out[:, 512:516]], axis=1)
        elif kind == "byte_swapped_rope":
            rope = out[:, 528:].reshape(-1, 64, 2)
            out[:, 528:] = rope[:, :, ::-1].reshape(-1, 128)
        elif kind in ("tiles_of_64", "one_scale"):
            from oracle import quantize

            values = fp8.bf16_bits_to_f32(bits[:, :512])
            width = 64 if kind == "tiles_of_64" else 512
            codes, scales = quantize.quantize_index(values.reshape(len(bits), -1, width))
            out[:, :512] = codes.reshape(len(bits), 512)
            tile_scales = np.repeat(scales.reshape(len(bits), -1), 512 // width // 4 or 1,
                                    axis=1)[:, ::max(1, 128 // width)][:, :4]
            if kind == "one_scale":
                tile_scales = np.repeat(scales.reshape(len(bits), 1), 4, axis=1)
            out[:, 512:528] = np.ascontiguousarray(tile_scales.astype("<f4")).view(np.uint8)
        return out

    return encode


@pytest.mark.parametrize("kind", ["swapped_scale_bytes", "swapped_tile_scales",
                                  "byte_swapped_rope", "tiles_of_64", "one_scale"])
def test_pins_reject_planted_mistakes(kind):
    encode = _mutant(kind)
    failures = 0
    for check in CHECKS:
        try:
            with np.errstate(all="ignore"):
                check(encode, _inputs(40, 0))
        except AssertionError:
            failures += 1
    assert failures > 0, f"no pin detects the planted mistake {kind!r}"
