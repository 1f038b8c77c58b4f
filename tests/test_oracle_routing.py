"""Pins oracle.routing: the sigmoid against float64 math, route() against transformers'
DeepseekV3TopkRouter (golden fixture), invariants and closed-form special cases."""
from pathlib import Path

import math

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


def _brute_topk(b_row, kept_groups, top_k=8, gsz=32):
    """kernel.py:515-534 as plain Python loops over one token: -inf outside the kept groups;
    each round scans all experts for the largest value, keeps the first index holding it,
    then sets that entry to -inf (so a chosen expert ties with every other -inf entry)."""
    pruned = [float(b_row[e]) if (e // gsz) in kept_groups else -math.inf for e in range(len(b_row))]
    ids = []
    for _ in range(top_k):
        best, arg = -math.inf, None
        for e, v in enumerate(pruned):
            if arg is None or v > best:
                best, arg = v, e
        ids.append(arg)
        pruned[arg] = -math.inf
    return ids


def _brute_groups(b_row, topk_group=4, n_group=8, gsz=32):
    """kernel.py:479-501 as loops: group score = max + max of the rest (first maximum masked);
    rounds of 'largest score among unselected groups, lowest index on ties'."""
    scores = []
    for g in range(n_group):
        vals = [float(v) for v in b_row[g * gsz:(g + 1) * gsz]]
        i1 = max(range(gsz), key=lambda i: (vals[i], -i))
        rest = [v for i, v in enumerate(vals) if i != i1]
        scores.append(np.float32(vals[i1]) + np.float32(max(rest)))
    kept = []
    for _ in range(topk_group):
        cand = [g for g in range(n_group) if g not in kept]
        kept.append(max(cand, key=lambda g: (scores[g], -g)))
    return set(kept)


FEW_FINITE = {
    0: [],
    1: [77],
    5: [3, 17, 40, 70, 100],
    7: [0, 1, 2, 33, 34, 64, 96],
    "mixed": [0, 1, 32, 64, 96, 128, 129, 160, 192, 193, 224],
}


@pytest.mark.parametrize("case", list(FEW_FINITE))
def test_route_fewer_than_top_k_finite_candidates(case):
    """Biases of -inf leave fewer than 8 finite biased scores in the kept groups. Then, as in
    kernel.py:522-534, the maximum of a later round is -inf and its first index, expert 0, wins,
    again in every later round: a token names one expert several times. Pinned by the loop restatement above and by closed forms."""
    rng = np.random.default_rng(31)
    logits = rng.standard_normal((40, 256)).astype(np.float32)
    bias = np.full(256, -np.inf, np.float32)
    fin = FEW_FINITE[case]
    bias[fin] = (rng.standard_normal(len(fin)) * 0.1).astype(np.float32)
    ids, w = routing.route(logits, bias, 2.5)
    b = routing.sigmoid_f32(logits) + bias
    s = routing.sigmoid_f32(logits)
    for t in range(logits.shape[0]):
        kept = _brute_groups(b[t])
        assert ids[t].tolist() == _brute_topk(b[t], kept)
        nfin = sum(1 for e in fin if e // 32 in kept)
        assert nfin < 8
        # closed form: the finite candidates first (descending b, lower index on ties), then
        # expert 0 in every remaining slot: by then every entry is -inf and 0 is the first index
        first = sorted((e for e in fin if e // 32 in kept), key=lambda e: (-b[t, e], e))
        assert ids[t, :nfin].tolist() == first
        assert ids[t, nfin:].tolist() == [0] * (8 - nfin)
        # weights: unbiased scores of the named experts, repeats included, over their sum
        sv = s[t, ids[t]].astype(np.float64)
        np.testing.assert_allclose(w[t], sv / sv.sum() * 2.5, rtol=3e-6)
    if case == 0:
        # all biased scores -inf: groups 0-3 kept, expert 0 eight times, weight rsf/8 at logit 0
        ids0, w0 = routing.route(np.zeros((2, 256), np.float32), bias, 2.5)
        assert ids0.tolist() == [[0] * 8] * 2
        assert np.all(w0 == np.float32(2.5 / 8))


def test_route_few_finite_repeats_are_lowest_index_of_kept_groups():
    """One finite expert (77, group 2): every group score is -inf (a group needs two finite
    entries), so groups 0-3 are kept on the lowest-index rule, and the seven remaining slots
    all name expert 0."""
    bias = np.full(256, -np.inf, np.float32)
    bias[77] = 0.0
    logits = np.random.default_rng(2).standard_normal((5, 256)).astype(np.float32)
    ids, _ = routing.route(logits, bias, 1.0)
    assert ids.tolist() == [[77] + [0] * 7] * 5
