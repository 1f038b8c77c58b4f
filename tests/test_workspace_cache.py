"""The per-stream workspace cache's retention policy (moe.WorkspaceCache), on the CPU with
an injected allocator and capture flag: a workspace that a graph capture used is never freed
when a larger call replaces it; one that no capture used is released."""
import gc
import weakref
from types import SimpleNamespace

import pytest


@pytest.fixture(scope="module")
def moe(pkg):
    from mlsys26_flashinfer_moe_amd import moe
    return moe


class _Ws:
    def __init__(self, T):
        self.buffer = SimpleNamespace(numel=lambda n=1000 * T: n)
        self.layout = SimpleNamespace(num_tokens=T)
        self.captured = False


def _cache(moe, flag):
    made = []

    def make(T, dev, stream):
        ws = _Ws(T)
        made.append(weakref.ref(ws))
        return ws

    return moe.WorkspaceCache(make=make, capturing=lambda: flag["on"]), made


def test_captured_workspace_survives_growth(moe):
    flag = {"on": True}
    cache, made = _cache(moe, flag)
    small = cache.get(("dev", 1), 16, 16000, None, None)
    assert small.captured
    flag["on"] = False
    big = cache.get(("dev", 1), 64, 64000, None, None)
    assert big is not small and not big.captured
    assert cache.retired == [small]
    del small, big
    gc.collect()
    assert made[0]() is not None, "the workspace a graph captured was freed"


def test_uncaptured_workspace_is_released_on_growth(moe):
    flag = {"on": False}
    cache, made = _cache(moe, flag)
    cache.get(("dev", 2), 16, 16000, None, None)
    cache.get(("dev", 2), 64, 64000, None, None)
    gc.collect()
    assert made[0]() is None and cache.retired == []


def test_reuse_same_stream_and_separate_streams(moe):
    flag = {"on": False}
    cache, made = _cache(moe, flag)
    a = cache.get(("dev", 3), 64, 64000, None, None)
    assert cache.get(("dev", 3), 64, 64000, None, None) is a
    assert cache.get(("dev", 3), 64, 10, None, None) is a        # a smaller call reuses it
    assert cache.get(("dev", 4), 64, 64000, None, None) is not a   # another stream: its own
    flag["on"] = True
    assert cache.get(("dev", 3), 64, 64000, None, None) is a and a.captured   # marked by a capture
