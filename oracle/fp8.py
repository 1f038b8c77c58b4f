"""OCP fp8 e4m3fn codec and bf16 rounding in numpy (oracle; test infrastructure only).

e4m3fn: 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 encodes
subnormals m/8 * 2^-6; exponent 15 with mantissa 7 is NaN; there are no infinities;
the largest finite value is 448. Encoding rounds to nearest, ties to even, and gives NaN
for |x| > 464 (values in (448, 464] round to 448) -- the semantics of torch's
float8_e4m3fn cast, which the Triton cast of kernel.py:135 also targets.
"""
from __future__ import annotations

import numpy as np


def _decode_table() -> np.ndarray:
    codes = np.arange(256, dtype=np.int64)
    sign = (codes >> 7) & 1
    exp = (codes >> 3) & 0xF
    man = codes & 7
    mag = np.where(exp == 0, man / 8.0 * 2.0 ** -6, (1.0 + man / 8.0) * np.exp2(exp - 7.0))
    val = np.where(sign == 1, -mag, mag)
    val = np.where((exp == 15) & (man == 7), np.nan, val)
    return val.astype(np.float32)


E4M3_TABLE = _decode_table()
E4M3_MAX = np.float32(448.0)


def decode(codes: np.ndarray) -> np.ndarray:
    """uint8 e4m3fn codes -> float32 values."""
    return E4M3_TABLE[np.asarray(codes, dtype=np.uint8)]


def encode(x: np.ndarray) -> np.ndarray:
    """float32 -> uint8 e4m3fn codes, round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    a = np.abs(x).astype(np.float64)
    sign = np.signbit(x).astype(np.uint16) << 7
    frac, e = np.frexp(a)                     # a = frac * 2^e, frac in [0.5, 1)
    sub = a < 2.0 ** -6
    # subnormal range: code = round(a / 2^-9); 8 becomes the smallest normal (code 8)
    code_sub = np.rint(a * 2.0 ** 9)
    # normal range: a = (2 frac) 2^(e-1); code = (E + 7) * 8 + round((2 frac - 1) * 8)
    code_norm = (e - 1 + 7) * 8 + np.rint((2.0 * frac - 1.0) * 8.0)
    code = np.where(sub, code_sub, code_norm)
    code = np.where(np.isnan(a) | (code >= 127), 127, code).astype(np.uint16)
    return (code | sign).astype(np.uint8)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> quiet NaN."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float32 -> float32 values rounded to bf16 (round to nearest even)."""
    return (bf16_bits(x).astype(np.uint32) << 16).view(np.float32)


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
