"""Pins oracle/experts.py (kernel.py:104-135, 228-234): exact small-integer cases, one-hot
rows, torch CPU matmul as the library routine for the GEMMs, the SwiGLU half convention in
closed form, and the requantisation's closed forms with torch's CPU fp8 cast."""
import math

import numpy as np
import torch

from oracle import experts as ex
from oracle import fp8 as ofp8


def _fp8_codes(values):
    return torch.tensor(np.asarray(values, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def test_dequant_rows_small_integers_exact():
    rng = np.random.default_rng(1)
    vals = rng.integers(-8, 9, (3, 256)).astype(np.float32)          # exactly representable in e4m3
    q = _fp8_codes(vals)
    scale = np.array([[0.5, 2.0, 4.0], [8.0, 0.25, 1.0]], np.float32)  # [K/128, n], powers of two
    a = ex.dequant_rows(q, scale)
    for t in range(3):
        for k in range(256):
            assert a[t, k] == vals[t, k] * scale[k // 128, t]


def test_dequant_blocks_small_integers_exact():
    rng = np.random.default_rng(2)
    vals = rng.integers(-6, 7, (256, 384)).astype(np.float32)
    q = _fp8_codes(vals)
    scale = (2.0 ** rng.integers(-4, 5, (2, 3))).astype(np.float32)
    w = ex.dequant_blocks(q, scale)
    expect = vals * np.repeat(np.repeat(scale, 128, 0), 128, 1)
    assert np.array_equal(w, expect)


def test_gemm_matches_torch_and_one_hot_selects_a_row():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 256)).astype(np.float32)
    w = rng.standard_normal((384, 256)).astype(np.float32)
    ref = (torch.from_numpy(x).double() @ torch.from_numpy(w).double().T).numpy()
    np.testing.assert_allclose(ex.gemm(x, w), ref, rtol=1e-5, atol=1e-4)
    onehot = np.zeros((1, 256), np.float32)
    onehot[0, 17] = 1.0
    assert np.array_equal(ex.gemm(onehot, w)[0], w[:, 17])
    # small integers: every product and partial sum is exact in fp32
    xi = rng.integers(-3, 4, (4, 256)).astype(np.float32)
    wi = rng.integers(-3, 4, (8, 256)).astype(np.float32)
    assert np.array_equal(ex.gemm(xi, wi), (xi.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32))


def test_swiglu_applies_silu_to_the_second_half():
    # g = [X1 | X2]; C = silu(X2) * X1 (kernel.py:126-129)
    x1 = np.array([[2.0, -3.0, 0.5, 7.0]], np.float32)
    x2 = np.array([[1.0, 0.0, -2.0, 30.0]], np.float32)
    c = ex.swiglu(np.concatenate([x1, x2], axis=1), 4)
    silu = lambda v: v / (1.0 + math.exp(-v))
    expect = [silu(float(b)) * float(a) for a, b in zip(x1[0], x2[0])]
    np.testing.assert_allclose(c[0], expect, rtol=2e-7, atol=0)
    assert c[0, 1] == 0.0                       # X2 = 0 gives C = 0 whatever X1 is
    # swapping the halves changes the result: the convention is not symmetric
    assert not np.allclose(ex.swiglu(np.concatenate([x2, x1], axis=1), 4), c)


def test_requant_rows_closed_forms():
    rng = np.random.default_rng(4)
    c = rng.standard_normal((3, 256)).astype(np.float32)
    c[1, :128] = 0.0                            # an all-zero block
    c[2, 5] = -1000.0                           # a negative block maximum
    q, sc = ex.requant_rows(c, 128)
    amax = np.abs(c.reshape(3, 2, 128)).max(-1)
    assert np.array_equal(sc, np.maximum((amax / np.float32(448.0)).astype(np.float32), np.float32(1e-12)))
    assert sc[1, 0] == np.float32(1e-12) and np.all(q[1, :128] == 0)
    # the element of largest magnitude lands on +-448 (code 0x7E / 0xFE) or one step below it
    assert q[2, 5] in (0xFE, 0xFD)
    # q is torch's fp8 cast of c / scale (division in fp32)
    ref = _fp8_codes((c.reshape(3, 2, 128) / sc[..., None]).astype(np.float32)).reshape(3, 256)
    assert np.array_equal(q, ref)
    # round trip: within half an fp8 step (2^-4 relative) or the subnormal spacing
    back = ex.dequant_requant(q, sc, 128)
    step = np.repeat(sc, 128, axis=1) * 2.0 ** -9
    assert np.all(np.abs(back - c) <= np.abs(c) * 2.0 ** -4 + step)


def test_requant_codes_match_decode_table():
    q, sc = ex.requant_rows(np.full((1, 128), 3.0, np.float32), 128)
    assert sc[0, 0] == np.float32(3.0 / 448.0)
    assert np.all(ofp8.decode(q) * sc[0, 0] == np.float32(448.0) * sc[0, 0])
