"""Pins oracle.routing: the sigmoid against float64 math, route() against transformers'
DeepseekV3TopkRouter (golden fixture), invariants and closed-form special cases."""
from pathlib import Path

import numpy as np
import pytest

from oracle import routing

GOLD = np.load(Path(__file__).parent / "golden" / "routing_golden.npz")


def test_constants_are_the_kernel_bit_patterns():
    bits = lambda v: int(np.float32(v).view(np.uint32))
    assert bits(routing.LOG2E) == 0x3FB8AA3B
    assert bits(routing.LN2_HI) == 0x3F318000
    assert bits(routing.LN2_LO) == 0xB95E8083
    assert [bits(c) for c in routing.TAYLOR[3:]] == [0x3E2AAAAB, 0x3D2AAAAB, 0x3C088889, 0x3AB60B61, 0x39500D01]
    # LN2_HI + LN2_LO is ln 2 to fp32 working precision
    assert abs(float(routing.LN2_HI) + float(routing.LN2_LO) - np.log(2.0)) < 1e-11


def test_sigmoid_accuracy_and_shape():
    x = np.linspace(-30, 30, 600001, dtype=np.float32)
    s = routing.sigmoid_f32(x)
    ref = 1.0 / (1.0 + np.exp(-x.astype(np.float64)))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(s - ref) / ulp) <= 3.0
    assert np.all(np.diff(s) >= 0)                         # monotone
    assert routing.sigmoid_f32(np.float32(0.0)) == 0.5
    sym = routing.sigmoid_f32(x) + routing.sigmoid_f32(-x)
    assert np.max(np.abs(sym - 1.0)) < 3e-7


def test_sigmoid_saturation():
    s = routing.sigmoid_f32(np.array([-1e30, -200, -80, 80, 200, 1e30, np.inf, -np.inf], np.float32))
    assert np.all(np.isfinite(s)) and np.all(s >= 0) and np.all(s <= 1)
    assert s[3] == 1.0 and s[4] == 1.0 and s[0] == s[1] == s[2] > 0


def _route_golden_part(i):
    m = GOLD["bias_index"] == i
    ids, w = routing.route(GOLD["logits"][m], GOLD["bias_sets"][i], float(GOLD["routed_scaling_factor"]))
    order = np.argsort(ids, axis=1)
    return m, np.take_along_axis(ids, order, 1), np.take_along_axis(w, order, 1)


@pytest.mark.parametrize("part", [0, 1, 2])
def test_route_matches_transformers_router(part):
    m, ids, w = _route_golden_part(part)
    assert np.array_equal(ids, GOLD["ids_sorted"][m])
    np.testing.assert_allclose(w, GOLD["weights_sorted"][m], rtol=2e-6, atol=0)


def test_route_invariants():
    rng = np.random.default_rng(3)
    logits = rng.standard_normal((300, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    ids, w = routing.route(logits, bias, 2.5)
    assert ids.shape == (300, 8) and ids.dtype == np.int32
    for row in ids:
        assert len(set(row.tolist())) == 8
        assert len(set((row // 32).tolist())) <= 4
    assert np.all(w >= 0)
    np.testing.assert_allclose(w.sum(axis=1), 2.5, rtol=2e-6)
    # selection order is descending biased score
    b = routing.sigmoid_f32(logits) + bias
    sel = np.take_along_axis(b, ids, 1)
    assert np.all(np.diff(sel, axis=1) <= 0)


def test_route_ties_pick_lowest_index():
    logits = np.zeros((3, 256), np.float32)
    bias = np.zeros(256, np.float32)
    ids, w = routing.route(logits, bias, 1.0)
    assert np.array_equal(ids, np.tile(np.arange(8, dtype=np.int32), (3, 1)))
    np.testing.assert_allclose(w, 1.0 / 8, rtol=1e-7)


def test_route_forced_by_bias():
    rng = np.random.default_rng(5)
    logits = rng.standard_normal((64, 256)).astype(np.float32)
    bias = np.zeros(256, np.float32)
    bias[[40, 77, 200, 201]] = 3.0
    ids, w = routing.route(logits, bias, 2.5)
    for row in ids:
        assert {40, 77, 200, 201} <= set(row.tolist())
        assert sorted(row[:4].tolist()) == [40, 77, 200, 201]


def test_route_bias_zero_is_topk_of_sigmoid_in_top_groups():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((50, 256)).astype(np.float32)
    ids, _ = routing.route(logits, np.zeros(256, np.float32), 1.0)
    s = 1.0 / (1.0 + np.exp(-logits.astype(np.float64)))
    g = np.sort(s.reshape(50, 8, 32), axis=-1)
    gscore = g[..., -1] + g[..., -2]
    for t in range(50):
        keep = np.argsort(-gscore[t], kind="stable")[:4]
        cand = np.concatenate([np.arange(32 * k, 32 * k + 32) for k in keep])
        best = cand[np.argsort(-s[t, cand], kind="stable")[:8]]
        assert set(best.tolist()) == set(ids[t].tolist())


def test_weights_use_unbiased_scores():
    # Lowering one selected expert's bias (without changing the selected set) changes the
    # selection order but not any expert's weight, which comes from the unbiased score.
    logits = np.full((1, 256), -5.0, np.float32)
    logits[0, :8] = np.arange(8, dtype=np.float32)
    bias = np.zeros(256, np.float32)
    ids0, w0 = routing.route(logits, bias, 2.5)
    bias[7] = -0.9
    ids1, w1 = routing.route(logits, bias, 2.5)
    assert set(ids0[0].tolist()) == set(ids1[0].tolist()) == set(range(8))
    assert list(ids1[0]).index(7) > list(ids0[0]).index(7)
    d0 = dict(zip(ids0[0].tolist(), w0[0].tolist()))
    d1 = dict(zip(ids1[0].tolist(), w1[0].tolist()))
    for e in range(8):
        assert abs(d0[e] - d1[e]) <= 2e-7 * d0[e]
    # weight ratio equals the ratio of unbiased scores
    s = 1.0 / (1.0 + np.exp(-np.arange(8.0)))
    np.testing.assert_allclose([d1[e] / d1[0] for e in range(8)], s / s[0], rtol=1e-6)
