"""OCP float8 e4m3fn codec in numpy (TEST INFRASTRUCTURE ONLY).

e4m3fn: 1 sign, 4 exponent (bias 7), 3 mantissa bits, no infinities, NaN is
S.1111.111, largest finite 448 (0x7E), smallest subnormal 2**-9. The encoder
rounds to nearest even; magnitudes >= 480 (the first value that would round
past 448) and NaN become 0x7F with the input sign, the behaviour of
``tensor.to(torch.float8_e4m3fn)``.

Pinned by: ``tests/test_oracle_fp8_quantize.py`` compares ``encode`` bit-for-bit with
torch's own float8 cast over every bf16 bit pattern, random fp32 values and all
e4m3 rounding midpoints, and ``decode`` with torch's float8->float32 cast over
all 256 codes.
"""

import numpy as np

_MIN_NORMAL_BITS = 0x3C800000  # 2**-6, smallest normal e4m3 magnitude
_OVERFLOW_BITS = 0x43F00000  # 480.0: rounds past 448, becomes NaN


def encode(x):
    """float32 array -> uint8 e4m3fn codes, round to nearest even."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    mag = bits & np.uint32(0x7FFFFFFF)
    out = np.zeros(x.shape, dtype=np.uint8)

    big = mag >= _OVERFLOW_BITS
    small = mag < _MIN_NORMAL_BITS
    normal = ~(big | small)

    # Subnormal range: value = m * 2**-9 with m in [0, 8]; m == 8 is the
    # smallest normal code 0x08, so the integer is the code itself.
    sub = np.rint(np.abs(x[small]) * np.float32(512.0)).astype(np.uint32)
    out[small] = sub.astype(np.uint8)

    # Normal range: keep 3 of 23 mantissa bits with round-half-even on the
    # dropped 20 bits, then rebias the exponent from 127 to 7.
    m = mag[normal]
    rounded = (m + np.uint32(0x7FFFF) + ((m >> 20) & np.uint32(1))) >> 20
    out[normal] = (rounded - np.uint32(120 << 3)).astype(np.uint8)

    out[big] = 0x7F
    return out | sign


def decode(codes):
    """uint8 e4m3fn codes -> float32 values (NaN for S.1111.111)."""
    c = np.asarray(codes, dtype=np.uint8).astype(np.int32)
    sign = np.where(c & 0x80, -1.0, 1.0)
    e = (c >> 3) & 0xF
    m = c & 7
    mag = np.where(e == 0, m * 2.0**-9, (1.0 + m / 8.0) * np.exp2(e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return (sign * mag).astype(np.float32)


def bf16_bits_to_f32(bits):
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    b = np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16
    return b.view(np.float32)


def f32_to_bf16_bits(x):
    """float32 -> bf16 bit patterns, round to nearest even; NaN -> 0x7FC0 (torch's)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    nan = np.isnan(x)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    out = rounded.astype(np.uint16)
    out[nan] = 0x7FC0
    return out
