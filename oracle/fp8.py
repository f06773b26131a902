"""OCP FP8 E4M3FN codec (test infrastructure only).

E4M3FN: 1 sign, 4 exponent (bias 7), 3 mantissa bits; max finite 448 (0x7E),
0x7F / 0xFF are NaN, no infinities, subnormals m * 2^-9.  This is the format
of ``torch.float8_e4m3fn`` and of Triton's ``float8e4nv`` used by the
reference (``quant_triton.py:57``, ``attention_triton.py:331``).

Encoding is round-to-nearest-even on the fp32 bits.  Every caller in the
reference clamps to [-448, 448] before the cast (``quant_triton.py:49``,
``attention_triton.py:344, 357``), or relies on Triton's ``satfinite``
conversion for elementwise P (``attention_triton.py:331``); ``encode``
therefore saturates finite inputs to +-448, which equals both behaviours.

Pinned by ``tests/test_oracle_fp8.py`` against ``torch.float8_e4m3fn`` on all
bf16 bit patterns (with several low-bit fills), every representable E4M3
value, every rounding midpoint and its fp32 neighbours, and the full decode
table.
"""

from __future__ import annotations

import numpy as np

FP8_MAX = 448.0


def encode(x) -> np.ndarray:
    """fp32 array -> uint8 E4M3FN codes (RNE, saturating to +-448)."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    u = x.view(np.uint32).astype(np.uint64)
    sign = (u >> 31) & 1
    a = u & 0x7FFFFFFF
    out = np.zeros(a.shape, dtype=np.uint64)

    nan = a > 0x7F800000
    big = (a >= 0x43E00000) & ~nan            # |x| >= 448 (incl. inf): saturate
    normal = (a >= 0x3C800000) & ~big & ~nan   # 2^-6 <= |x| < 448
    sub = a < 0x3C800000                       # |x| < 2^-6

    # normal range: keep 3 mantissa bits, RNE on the 20 dropped bits
    e = (a >> 23).astype(np.int64) - 127
    mant = a & 0x7FFFFF
    q = mant >> 20
    rem = mant & 0xFFFFF
    up = (rem > 0x80000) | ((rem == 0x80000) & ((q & 1) == 1))
    q = q + up.astype(np.uint64)
    carry = q == 8
    q = np.where(carry, 0, q)
    e = e + carry.astype(np.int64)
    code_n = (((e + 7).astype(np.uint64)) << 3) | q
    # (e+7, q) == (15, 7) would be 480 -> impossible for |x| < 448 (448 = 15,6;
    # values in (448, 464) round to 448, [464, 480) can only come from |x|>=448).
    out = np.where(normal, code_n, out)

    # subnormal range: value * 2^9 rounded to an integer 0..8 (8 == min normal)
    E = (a >> 23).astype(np.int64)
    M = np.where(E > 0, (a & 0x7FFFFF) | 0x800000, a & 0x7FFFFF).astype(np.uint64)
    Eeff = np.where(E > 0, E, 1)
    shift = (141 - Eeff).astype(np.uint64)     # value*2^9 = M * 2^(Eeff-141)
    shift_c = np.minimum(shift, 63)
    qs = M >> shift_c
    dropped = M - (qs << shift_c)
    half = np.where(shift_c > 0, np.uint64(1) << (shift_c - 1), 0)
    ups = (dropped > half) | ((dropped == half) & (half > 0) & ((qs & 1) == 1))
    qs = np.where(shift > 62, 0, qs + ups.astype(np.uint64))
    out = np.where(sub, qs, out)

    out = np.where(big, 0x7E, out)
    out = np.where(nan, 0x7F, out)
    out = out | (sign << 7)
    return out.astype(np.uint8)


def _decode_table() -> np.ndarray:
    t = np.zeros(256, dtype=np.float32)
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 7
        if e == 15 and m == 7:
            t[c] = np.nan
        elif e == 0:
            t[c] = s * m * 2.0 ** -9
        else:
            t[c] = s * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return t


DECODE = _decode_table()


def decode(codes) -> np.ndarray:
    """uint8 E4M3FN codes -> fp32 values."""
    return DECODE[np.asarray(codes, dtype=np.uint8)]


def round_to_e4m3(x) -> np.ndarray:
    """fp32 -> nearest E4M3 value (saturating), returned as fp32."""
    return decode(encode(x))
