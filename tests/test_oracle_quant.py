"""The oracle of the upstream activation quantiser (oracle/quant.py), pinned against
torch's CPU float8_e4m3fn cast and closed forms. CPU only."""
import numpy as np
import pytest
import torch

from oracle import fp8, quant

H = 7168


def _data(T, seed, dtype=np.float32, emin=-30, emax=30):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((T, H)).astype(np.float32)
    # per-block magnitudes 2^emin .. 2^emax; the smallest blocks hit the 1e-12 scale clamp
    mag = np.exp2(rng.integers(emin, emax + 1, size=(T, H // 128))).astype(np.float32)
    return (x.reshape(T, H // 128, 128) * mag[..., None]).reshape(T, H).astype(dtype)


@pytest.mark.parametrize("T", [1, 3, 40])
def test_matches_torch_cpu_cast(T):
    x = _data(T, 100 + T)
    q, s = quant.quantize_hidden(x)
    xt = torch.from_numpy(x).reshape(T, H // 128, 128)
    st = torch.clamp_min(xt.abs().amax(dim=-1) / 448.0, 1e-12)
    qt = (xt / st[..., None]).to(torch.float8_e4m3fn).view(torch.uint8).reshape(T, H)
    assert np.array_equal(q, qt.numpy())
    assert np.array_equal(s, st.t().contiguous().numpy())
    assert s.shape == (H // 128, T) and s.dtype == np.float32 and q.dtype == np.uint8


def test_block_max_is_448_and_zero_blocks():
    x = _data(4, 7)
    x[1, 128:256] = 0.0
    x[2, 0:128] = -0.0
    q, s = quant.quantize_hidden(x)
    v = fp8.decode(q).reshape(4, H // 128, 128)
    amax = np.abs(v).max(axis=-1)
    nonzero = np.abs(x).reshape(4, H // 128, 128).max(axis=-1) > 0
    assert np.all(amax[nonzero] == 448.0)
    assert s[1, 1] == np.float32(1e-12) and s[0, 2] == np.float32(1e-12)
    assert not q[1, 128:256].any()
    assert np.all(q[2, 0:128] == 0x80)   # -0.0 keeps its sign


def test_power_of_two_scaling_and_sign_symmetry():
    x = _data(3, 11, emin=-20, emax=20)   # the 2^k-scaled scales stay above the 1e-12 clamp
    q, s = quant.quantize_hidden(x)
    for k in (-5, 3, 9):
        qk, sk = quant.quantize_hidden(x * np.float32(2.0 ** k))
        assert np.array_equal(qk, q)
        assert np.array_equal(sk, s * np.float32(2.0 ** k))
    qn, sn = quant.quantize_hidden(-x)
    assert np.array_equal(sn, s)
    assert np.array_equal(qn, q ^ 0x80)


def test_round_trip_error_bound():
    x = _data(8, 21)
    q, s = quant.quantize_hidden(x)
    scale = np.repeat(s.T, 128, axis=1)
    y = fp8.decode(q) * scale
    r = np.abs(x) / scale    # magnitude in units of the block scale (<= 448)
    err = np.abs(y - x) / scale
    # e4m3: half an ulp is 2^-4 relative for normals (>= 2^-6) and 2^-10 absolute below
    assert np.all(err <= np.maximum(r * 2.0 ** -4, 2.0 ** -10) * (1 + 1e-6))


def test_hidden_values_of_each_dtype():
    x = _data(2, 5)
    bits = fp8.bf16_bits(x)
    assert np.array_equal(quant.hidden_values(bits, "bf16"), fp8.bf16_round(x))
    assert np.array_equal(quant.hidden_values(x.astype(np.float16), "fp16"), x.astype(np.float16).astype(np.float32))
    assert np.array_equal(quant.hidden_values(x, "fp32"), x)
