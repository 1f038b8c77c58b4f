"""Pins oracle/dispatch.py: brute-force bucket construction, the reference's tile schedule
restated as loops, hand-worked work lists, and the invariants of kernel.py:327-407."""
import numpy as np
import pytest

from oracle import dispatch as odsp


def _brute_dispatch(ids, w, offset, e_local=32):
    """Loops over experts, then tokens, then top-k slots: the stable bucket order."""
    T, K = ids.shape
    buckets = [[] for _ in range(e_local)]
    for e in range(e_local):
        for t in range(T):
            for k in range(K):
                if int(ids[t, k]) - offset == e:
                    buckets[e].append(t * K + k)
    slots = [s for b in buckets for s in b]
    counts = [len(b) for b in buckets]
    start = [0]
    for c in counts:
        start.append(start[-1] + c)
    nlocal = [sum(1 for k in range(K) if 0 <= int(ids[t, k]) - offset < e_local) for t in range(T)]
    return slots, counts, start, nlocal


@pytest.mark.parametrize("T,offset,seed", [(1, 0, 0), (7, 32, 1), (33, 224, 2), (100, 0, 3), (64, -5, 4)])
def test_dispatch_matches_brute_force(T, offset, seed):
    rng = np.random.default_rng(seed)
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    if T > 3:
        ids[3, 1] = ids[3, 0]            # a repeated expert in one token's list
    w = rng.random((T, 8)).astype(np.float32)
    d = odsp.dispatch(ids, w, offset)
    slots, counts, start, nlocal = _brute_dispatch(ids, w, offset)
    assert d["sorted_slot"].tolist() == slots
    assert d["expert_count"].tolist() == counts
    assert d["expert_start"].tolist() == start
    assert d["token_nlocal"].tolist() == nlocal
    assert d["sorted_token"].tolist() == [s // 8 for s in slots]
    assert d["sorted_weight"].view(np.uint32).tolist() == [int(w.reshape(-1).view(np.uint32)[s]) for s in slots]


def test_dispatch_invariants():
    rng = np.random.default_rng(11)
    T = 500
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    w = rng.random((T, 8)).astype(np.float32)
    d = odsp.dispatch(ids, w, 64)
    n = int(d["expert_start"][-1])
    assert n == int(((ids >= 64) & (ids < 96)).sum()) == int(d["expert_count"].sum())
    assert np.all(np.diff(d["expert_start"]) >= 0) and d["expert_start"][0] == 0
    # every (token, local expert) pair exactly once, inside its expert's bucket
    pairs = set()
    for e in range(32):
        for r in range(d["expert_start"][e], d["expert_start"][e + 1]):
            s = int(d["sorted_slot"][r])
            assert ids.reshape(-1)[s] - 64 == e
            pairs.add((s // 8, e))
    assert len(pairs) == n


def test_dispatch_nothing_local():
    ids = np.full((4, 8), 200, dtype=np.int32)
    d = odsp.dispatch(ids, np.ones((4, 8), np.float32), 0)
    assert d["expert_start"].tolist() == [0] * 33
    assert len(d["sorted_slot"]) == 0 and d["token_nlocal"].tolist() == [0, 0, 0, 0]


def _brute_tiles(counts, bm):
    ex, lm = [], []
    for e, n in enumerate(counts):
        m = 0
        while m * bm < n:
            ex.append(e)
            lm.append(m)
            m += 1
    return ex, lm


@pytest.mark.parametrize("bm", [16, 64, 128])
def test_tile_schedule_matches_loops(bm):
    rng = np.random.default_rng(bm)
    counts = rng.integers(0, 300, 32)
    counts[[0, 5, 31]] = 0
    ex, lm, total = odsp.tile_schedule(counts, bm)
    bex, blm = _brute_tiles(counts.tolist(), bm)
    assert ex.tolist() == bex and lm.tolist() == blm and total == len(bex)
    assert total == int(sum((c + bm - 1) // bm for c in counts))


def test_work_items_hand_worked():
    counts = np.zeros(32, np.int32)
    counts[1], counts[2], counts[3] = 5, 40, 129
    start = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    # 16 rows per item: plain cuts
    got = odsp.work_items(counts, start, 16).tolist()
    assert got == [[1, 0, 5, 0 | 1 << 16],
                   [2, 5, 16, 1 | 3 << 16], [2, 21, 16, 1 | 3 << 16], [2, 37, 8, 1 | 3 << 16]] + \
                  [[3, 45 + 16 * i, 16, 4 | 9 << 16] for i in range(8)] + [[3, 173, 1, 4 | 9 << 16]]
    # 128 rows per item: balanced runs, a multiple of 16 rows (129 -> 2 runs of 80 + 49)
    got = odsp.work_items(counts, start, 128).tolist()
    assert got == [[1, 0, 5, 0 | 1 << 16], [2, 5, 40, 1 | 1 << 16],
                   [3, 45, 80, 2 | 2 << 16], [3, 125, 49, 2 | 2 << 16]]


@pytest.mark.parametrize("rpi", [16, 32, 128])
def test_work_items_cover_every_row_once(rpi):
    rng = np.random.default_rng(rpi + 5)
    counts = rng.integers(0, 700, 32).astype(np.int32)
    counts[::7] = 0
    start = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    items = odsp.work_items(counts, start, rpi)
    cover = np.zeros(int(start[-1]), np.int32)
    for i, (e, r0, rows, w) in enumerate(items):
        assert 0 < rows <= rpi and start[e] <= r0 and r0 + rows <= start[e + 1]
        first, nch = w & 0xFFFF, w >> 16
        assert first <= i < first + nch and items[first][0] == e
        cover[r0:r0 + rows] += 1
    assert np.all(cover == 1)
