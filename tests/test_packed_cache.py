"""CPU tests of the packed-weight cache behind run() (PackedWeightCache): when a copy is built,
reused, rebuilt or skipped, with the packing itself and the capture state injected."""
import gc

import pytest
import torch

import __graft_entry__ as ge


@pytest.fixture(scope="module")
def moe():
    ge.load_package()
    from mlsys26_flashinfer_moe_amd import moe
    return moe


class Recorder:
    def __init__(self):
        self.built = []
        self.capturing = False

    def make(self, w13, w2):
        p = torch.zeros(4)
        self.built.append(p)
        return p


def _cache(moe, rec, max_sets=2):
    rec.stream = 1
    rec.recorded = []
    rec.events = []
    rec.waited = []

    def event():
        ev = ("event", len(rec.events), rec.stream)   # an event recorded on the current stream
        rec.events.append(ev)
        return ev

    return moe.PackedWeightCache(max_sets=max_sets, make=rec.make, capturing=lambda: rec.capturing,
                                 stream_id=lambda: rec.stream, record=lambda p: rec.recorded.append((p, rec.stream)),
                                 event=event, wait=lambda ev: rec.waited.append((ev, rec.stream)))


def _set():
    return torch.zeros(64, dtype=torch.uint8), torch.zeros(32, dtype=torch.uint8)


def test_built_once_and_reused(moe):
    rec = Recorder()
    c = _cache(moe, rec)
    w13, w2 = _set()
    p = c.get(w13, w2)
    assert p is rec.built[0] and c.get(w13, w2) is p and len(rec.built) == 1
    # another view of the same storage at the same address is the same weight set
    assert c.get(w13.view(8, 8), w2) is p


def test_in_place_change_rebuilds(moe):
    rec = Recorder()
    c = _cache(moe, rec)
    w13, w2 = _set()
    p = c.get(w13, w2)
    w2.add_(1)
    q = c.get(w13, w2)
    assert q is not p and len(rec.built) == 2 and len(c) == 1
    assert c.retired == []           # no capture used the old copy: it is dropped


def test_full_cache_runs_row_major_without_eviction(moe):
    rec = Recorder()
    c = _cache(moe, rec, max_sets=2)
    sets = [_set() for _ in range(3)]
    a, b = c.get(*sets[0]), c.get(*sets[1])
    assert c.get(*sets[2]) is None and len(rec.built) == 2
    assert c.get(*sets[0]) is a and c.get(*sets[1]) is b


def test_freed_weights_free_their_slot(moe):
    rec = Recorder()
    c = _cache(moe, rec, max_sets=1)
    w13, w2 = _set()
    c.get(w13, w2)
    del w13, w2
    gc.collect()
    x13, x2 = _set()
    assert c.get(x13, x2) is rec.built[1] and len(c) == 1


def test_no_copy_is_built_under_capture_and_captured_copies_are_kept(moe):
    rec = Recorder()
    c = _cache(moe, rec)
    w13, w2 = _set()
    rec.capturing = True
    assert c.get(w13, w2) is None and rec.built == []
    rec.capturing = False
    p = c.get(w13, w2)
    rec.capturing = True
    assert c.get(w13, w2) is p       # a capture records the copy's address...
    rec.capturing = False
    w13.add_(1)
    q = c.get(w13, w2)
    assert q is not p and c.retired == [p]   # ...so the stale copy stays alive


def test_off_and_clear(moe):
    rec = Recorder()
    c = _cache(moe, rec, max_sets=0)
    assert c.get(*_set()) is None and rec.built == []
    c.max_sets = 2
    w13, w2 = _set()
    c.get(w13, w2)
    c.clear()
    assert len(c) == 0 and c.get(w13, w2) is rec.built[1]


def test_other_streams_are_recorded_once(moe):
    """A copy used on a stream other than its builder's is recorded there (record_stream) once, so
    that dropping it never frees memory that work queued on that stream may still read."""
    rec = Recorder()
    c = _cache(moe, rec)
    w13, w2 = _set()
    p = c.get(w13, w2)             # built on stream 1: nothing to record
    assert c.get(w13, w2) is p and rec.recorded == []
    rec.stream = 2
    assert c.get(w13, w2) is p and rec.recorded == [(p, 2)]
    c.get(w13, w2)
    rec.stream = 1
    c.get(w13, w2)
    assert rec.recorded == [(p, 2)]
    # a rebuilt copy starts over on the stream that builds it
    w13.add_(1)
    rec.stream = 3
    q = c.get(w13, w2)
    assert q is not p and rec.recorded == [(p, 2)]
    rec.stream = 1
    assert c.get(w13, w2) is q and rec.recorded == [(p, 2), (q, 1)]


def test_other_streams_wait_for_the_build_once(moe):
    """The packing kernel runs on the building stream. A stream that later reads the copy first
    waits for the event recorded right after that kernel (once per stream and copy), so that its
    GEMMs never read the copy before it is written; under capture no wait is added."""
    rec = Recorder()
    c = _cache(moe, rec)
    w13, w2 = _set()
    p = c.get(w13, w2)
    assert rec.events == [("event", 0, 1)] and rec.waited == []
    assert c.get(w13, w2) is p and rec.waited == []          # the building stream is ordered already
    rec.stream = 2
    assert c.get(w13, w2) is p and rec.waited == [(("event", 0, 1), 2)]
    c.get(w13, w2)
    rec.stream = 1
    c.get(w13, w2)
    assert rec.waited == [(("event", 0, 1), 2)]
    rec.stream, rec.capturing = 3, True
    assert c.get(w13, w2) is p and rec.waited == [(("event", 0, 1), 2)]
    assert rec.recorded == [(p, 2), (p, 3)]
    # a rebuilt copy has its own event, waited for by the other streams again
    rec.capturing = False
    w13.add_(1)
    q = c.get(w13, w2)
    rec.stream = 2
    assert c.get(w13, w2) is q and rec.waited[-1] == (rec.events[-1], 2) and len(rec.events) == 2


def test_a_copy_that_does_not_fit_runs_row_major(moe):
    """An out-of-memory error while allocating the copy leaves run() on the row-major weights
    (no extra memory); the set is not tried again until clear()."""
    rec = Recorder()
    calls = []

    def make(w13, w2):
        calls.append(1)
        raise torch.cuda.OutOfMemoryError("no room for the packed copy")

    c = _cache(moe, rec)
    c._make = make
    w13, w2 = _set()
    assert c.get(w13, w2) is None and c.get(w13, w2) is None
    assert len(calls) == 1 and len(c) == 0 and rec.events == []
    c.clear()
    c._make = rec.make
    assert c.get(w13, w2) is rec.built[0]
