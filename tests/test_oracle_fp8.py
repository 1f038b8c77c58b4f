"""Pins oracle.fp8 against torch's CPU casts (golden fixture) and the format definition."""
from pathlib import Path

import numpy as np

from oracle import fp8

GOLD = np.load(Path(__file__).parent / "golden" / "fp8_e4m3fn_golden.npz")


def test_decode_table_matches_torch():
    t = GOLD["decode_table"]
    assert np.array_equal(np.isnan(fp8.E4M3_TABLE), np.isnan(t))
    ok = ~np.isnan(t)
    assert np.array_equal(fp8.E4M3_TABLE[ok], t[ok])
    # signed zeros and NaN codes
    assert np.signbit(fp8.E4M3_TABLE[0x80]) and fp8.E4M3_TABLE[0x80] == 0
    assert np.isnan(fp8.E4M3_TABLE[0x7F]) and np.isnan(fp8.E4M3_TABLE[0xFF])


def test_format_closed_forms():
    assert fp8.E4M3_TABLE[0x7E] == 448.0          # largest finite
    assert fp8.E4M3_TABLE[0x01] == 2.0 ** -9      # smallest subnormal
    assert fp8.E4M3_TABLE[0x08] == 2.0 ** -6      # smallest normal
    assert fp8.E4M3_TABLE[0x38] == 1.0            # exponent bias 7
    # round trip of every finite code
    codes = np.arange(256, dtype=np.uint8)
    fin = np.isfinite(fp8.E4M3_TABLE)
    back = fp8.encode(fp8.E4M3_TABLE[fin])
    assert np.array_equal(back[fp8.E4M3_TABLE[fin] != 0], codes[fin][fp8.E4M3_TABLE[fin] != 0])


def test_encode_matches_torch_on_golden_values():
    got = fp8.encode(GOLD["values"])
    exp = GOLD["codes"]
    nan_exp = np.isnan(fp8.E4M3_TABLE[exp])
    assert np.array_equal(np.isnan(fp8.E4M3_TABLE[got]), nan_exp)
    assert np.array_equal(got[~nan_exp], exp[~nan_exp])


def test_encode_ties_to_even():
    # 1 + 1/16 lies halfway between 1 (mantissa 0) and 1.125 (mantissa 1): rounds to even 1.0
    assert fp8.decode(fp8.encode(np.float32(1.0625))) == 1.0
    # 1.1875 lies between 1.125 (m=1) and 1.25 (m=2): rounds to 1.25
    assert fp8.decode(fp8.encode(np.float32(1.1875))) == 1.25
    assert fp8.decode(fp8.encode(np.float32(464.0))) == 448.0
    assert np.isnan(fp8.decode(fp8.encode(np.float32(465.0))))


def test_bf16_rounding_matches_torch():
    assert np.array_equal(fp8.bf16_bits(GOLD["bf16_values"]), GOLD["bf16_bits"])
    # ties to even, closed form
    x = np.array([0x3F808000, 0x3F818000], dtype=np.uint32).view(np.float32)
    assert list(fp8.bf16_bits(x)) == [0x3F80, 0x3F82]


def test_bf16_to_f32_matches_torch():
    """Every bf16 bit pattern widens to torch's CPU bfloat16 -> float32 value (NaNs as NaN)."""
    import torch
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = fp8.bf16_to_f32(bits)
    exp = torch.from_numpy(bits.view(np.int16)).view(torch.bfloat16).float().numpy()
    nan = np.isnan(exp)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), exp[~nan].view(np.uint32))
