"""Pins oracle/layer.py (kernel.py:562-729): a pure-Python float64 brute force of the whole
composition (per token, per top-k slot: dequantise, GEMM1, SwiGLU, [fp8 requantisation with
torch's CPU cast], GEMM2, weight, accumulate) on tiny shapes."""
import math

import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import layer as olayer

H, I, E_L, OFF = 256, 128, 4, 8


def _codes(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def _decode64(q):
    return torch.from_numpy(np.ascontiguousarray(q)).view(torch.float8_e4m3fn).double().numpy()


def _inputs(T, seed):
    rng = np.random.default_rng(seed)
    hidden = _codes(rng.standard_normal((T, H)) * 40)
    hscale = (rng.random((H // 128, T)) * 0.05 + 0.01).astype(np.float32)
    w13 = _codes(rng.standard_normal((E_L, 2 * I, H)) * 30)
    s13 = (rng.random((E_L, 2 * I // 128, H // 128)) * 0.004 + 0.001).astype(np.float32)
    w2 = _codes(rng.standard_normal((E_L, H, I)) * 30)
    s2 = (rng.random((E_L, H // 128, I // 128)) * 0.004 + 0.001).astype(np.float32)
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    ids[0, :3] = [OFF + 2, OFF, OFF + 3]        # token 0: three local experts, out of order
    ids[1] = np.arange(100, 108)                # token 1: none local
    ids[2, 5] = OFF + 1                         # token 2: one local expert (maybe more)
    w = (rng.random((T, 8)) + 0.1).astype(np.float32)
    logits = rng.standard_normal((T, 256)).astype(np.float32)
    bias = np.zeros(256, np.float32)
    return dict(routing_logits=logits, routing_bias=bias, hidden_states=hidden, hidden_states_scale=hscale,
                gemm1_weights=w13, gemm1_weights_scale=s13, gemm2_weights=w2, gemm2_weights_scale=s2,
                local_expert_offset=OFF, routed_scaling_factor=2.5), (ids, w)


def _brute(kw, topk, requant_block=None):
    ids, w = topk
    T = ids.shape[0]
    out = np.zeros((T, H))
    for t in range(T):
        a = [_decode64(kw["hidden_states"][t, k:k + 1])[0] * float(kw["hidden_states_scale"][k // 128, t])
             for k in range(H)]
        for k in range(8):
            e = int(ids[t, k]) - OFF
            if not 0 <= e < E_L:
                continue
            w13 = _decode64(kw["gemm1_weights"][e]) * np.repeat(np.repeat(kw["gemm1_weights_scale"][e], 128, 0), 128, 1)
            g = [sum(w13[r, j] * a[j] for j in range(H)) for r in range(2 * I)]
            c = [g[i] * (g[I + i] / (1.0 + math.exp(-g[I + i]))) for i in range(I)]
            if requant_block:
                c32 = np.array(c, np.float32)
                for b0 in range(0, I, requant_block):
                    blk = c32[b0:b0 + requant_block]
                    sc = max(np.float32(np.abs(blk).max()) / np.float32(448.0), np.float32(1e-12))
                    q = _codes((blk / np.float32(sc)).astype(np.float32))
                    c[b0:b0 + requant_block] = list(_decode64(q) * float(sc))
            w2 = _decode64(kw["gemm2_weights"][e]) * np.repeat(np.repeat(kw["gemm2_weights_scale"][e], 128, 0), 128, 1)
            o = [sum(w2[h, i] * c[i] for i in range(I)) for h in range(H)]
            out[t] += float(w[t, k]) * np.array(o)
    return out


@pytest.mark.parametrize("seed", [0, 1])
def test_definition_mode_matches_brute_force(seed):
    kw, topk = _inputs(4, seed)
    r = olayer.layer_forward(**kw, mode="definition", topk=topk)
    ref = _brute(kw, topk)
    scale = np.abs(ref).max()
    np.testing.assert_allclose(r["output_f32"], ref, rtol=1e-4, atol=1e-5 * scale)
    assert np.array_equal(r["output"], ofp8.bf16_round(r["output_f32"]))
    assert np.all(r["output_f32"][1] == 0)      # no local expert -> exact zeros


def test_emulated_mode_matches_brute_force_with_torch_cast():
    kw, topk = _inputs(4, 2)
    r = olayer.layer_forward(**kw, mode="emulated", requant_block=64, topk=topk)
    ref = _brute(kw, topk, requant_block=64)
    scale = np.abs(ref).max()
    # fp32 vs float64 GEMM1 sums can flip a rare fp8 rounding of the intermediate
    err = np.abs(r["output_f32"] - ref)
    assert np.mean(err > 1e-3 * scale) < 0.01 and err.max() < 0.05 * scale
    # fp8 requantisation noise is a few per cent of each expert's contribution (the rows
    # of one token can cancel, so the yardstick is the per-assignment rows)
    d = olayer.layer_forward(**kw, mode="definition", topk=topk)
    assert np.sqrt(np.mean((r["rows"] - d["rows"]) ** 2)) < 0.05 * np.sqrt(np.mean(d["rows"] ** 2))


def test_tokens_subset_gives_the_same_rows():
    kw, topk = _inputs(5, 3)
    full = olayer.layer_forward(**kw, mode="definition", topk=topk)
    sub = olayer.layer_forward(**kw, mode="definition", topk=topk, tokens=np.array([0, 3]))
    assert np.array_equal(sub["output_f32"], full["output_f32"][[0, 3]])


def test_dequant_cache_gives_the_same_result():
    """A shared dequantisation cache across calls and modes changes no bit of the output."""
    kw, topk = _inputs(5, 4)
    cache = {}
    for mode in ("definition", "emulated"):
        plain = olayer.layer_forward(**kw, mode=mode, topk=topk)
        cached = olayer.layer_forward(**kw, mode=mode, topk=topk, dequant_cache=cache)
        assert np.array_equal(plain["output_f32"], cached["output_f32"])
    assert len(cache) > 0


@pytest.mark.parametrize("requant_block", [64, 128])
def test_act_override_reproduces_emulated_mode(requant_block):
    """GEMM2 + combine on a given intermediate: fed the emulated mode's own fp8 intermediate,
    the result is bit-identical; a changed intermediate byte, or a changed scale of the row's
    last block, changes the output of (only) the tokens whose rows use it."""
    kw, topk = _inputs(5, 5)
    ref = olayer.layer_forward(**kw, mode="emulated", topk=topk, requant_block=requant_block)
    act, sc = ref["act"].copy(), ref["act_scale"].copy()
    assert sc.shape[1] == kw["gemm2_weights"].shape[2] // requant_block
    got = olayer.layer_forward(**kw, mode="emulated", topk=topk, act_override=(act, sc),
                               requant_block=requant_block)
    assert np.array_equal(got["output_f32"], ref["output_f32"])
    row = 0
    tok = int(ref["sorted_token"][row])
    act[row, 3] ^= 0x01                          # one code step
    moved = olayer.layer_forward(**kw, mode="emulated", topk=topk, act_override=(act, sc),
                                 requant_block=requant_block)
    diff = np.any(moved["output_f32"] != ref["output_f32"], axis=1)
    assert diff[tok] and diff.sum() == 1
    act[row, 3] ^= 0x01
    sc[row, -1] *= 2.0                           # the row's last requant_block columns
    moved = olayer.layer_forward(**kw, mode="emulated", topk=topk, act_override=(act, sc),
                                 requant_block=requant_block)
    diff = np.any(moved["output_f32"] != ref["output_f32"], axis=1)
    assert diff[tok] and diff.sum() == 1
    with pytest.raises(ValueError):
        olayer.layer_forward(**kw, mode="definition", topk=topk, act_override=(act, sc))


@pytest.mark.parametrize("mode", ["definition", "emulated"])
def test_repeated_expert_in_one_token(mode):
    """A token may name one local expert several times (kernel.py:522-534 repeats expert 0 once
    fewer than 8 finite scores remain); each slot's weighted row is added, as the reference's
    per-slot scatter (kernel.py:313-321) and atomic add (kernel.py:246-250) do."""
    kw, (ids, w) = _inputs(3, 6)
    ids[0] = [OFF + 1, OFF + 3, 100, 101, 102, OFF, OFF, OFF]
    ids[2, :3] = [OFF + 2, OFF + 2, 50]
    r = olayer.layer_forward(**kw, mode=mode, topk=(ids, w), requant_block=64)
    ref = _brute(kw, (ids, w), requant_block=64 if mode == "emulated" else None)
    scale = np.abs(ref).max()
    err = np.abs(r["output_f32"] - ref)
    if mode == "definition":
        np.testing.assert_allclose(r["output_f32"], ref, rtol=1e-4, atol=1e-5 * scale)
    else:
        assert np.mean(err > 1e-3 * scale) < 0.01 and err.max() < 0.05 * scale
    assert r["token_nlocal"][0] == 5 and r["token_nlocal"][2] >= 2
