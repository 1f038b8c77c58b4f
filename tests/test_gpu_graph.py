"""The layer captured in a HIP graph (torch.cuda.CUDAGraph) replays to the eager result.

One call issues a fixed sequence of kernel launches for a given T, with no host
synchronisation, allocation or memset, so it can be captured once and replayed. Every replay
is checked bit for bit against an eager call on the same inputs, with eager work and
synchronisations between replays, and after the inputs' contents change in place.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _gh():
    import gpu_helpers
    return gpu_helpers


# decode path (stream GEMMs; at T=2 GEMM1's 6-slot ring, boosted local experts giving it work)
# and tile path
@pytest.mark.parametrize("T", [2, 48, 700])
def test_graph_replays_match_eager(T):
    gh = _gh()
    dev = torch.device("cuda:0")
    torch.manual_seed(T)
    w = gh.inputs.make_weights(31 + T, dev)
    boosted = (1, 7, 12, 30) if T <= 8 else ()
    logits, bias, hq, hs = gh.inputs.make_activations(T, 500 + T, dev, boosted_local_experts=boosted)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=0, routed_scaling_factor=2.5)
    side = torch.cuda.Stream(dev)
    out_eager = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    out_graph = torch.empty_like(out_eager)

    def eager():
        # the inputs are written on the default stream; the side stream must see them
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            gh.pkg.run(**kw, output=out_eager)
        side.synchronize()
        return out_eager.clone()

    print(f"graph capture T={T}", flush=True)
    ref = eager()   # also creates and initialises the workspace of `side` outside the capture
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    with torch.cuda.graph(g, stream=side):
        gh.pkg.run(**kw, output=out_graph)
    for rep in range(3):
        out_graph.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_graph, ref), f"replay {rep} differs from the eager result"
        # unrelated eager work between replays
        _ = (torch.randn(1 << 20, device=dev) * 2).sum().item()
    # new input contents, same tensors: the graph must read them
    kw["routing_logits"].copy_(torch.randn_like(kw["routing_logits"]))
    ref2 = eager()
    assert not torch.equal(ref2, ref)
    out_graph.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_graph, ref2)


def _kw(gh, T, seed, w):
    dev = torch.device("cuda:0")
    logits, bias, hq, hs = gh.inputs.make_activations(T, seed, dev)
    return dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
                gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
                local_expert_offset=0, routed_scaling_factor=2.5)


def _eager_on(stream, gh, kw, T):
    dev = torch.device("cuda:0")
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    stream.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(stream):
        gh.pkg.run(**kw, output=out)
    stream.synchronize()
    return out


def test_first_call_under_capture():
    """run() called for the first time inside torch.cuda.graph (its own capture stream, on which
    no call has run before): the workspace is allocated and initialised inside the capture by a
    kernel, and every replay equals an eager call."""
    gh = _gh()
    dev = torch.device("cuda:0")
    T = 24
    w = gh.inputs.make_weights(4100, dev)
    kw = _kw(gh, T, 4101, w)
    ref = _eager_on(torch.cuda.Stream(dev), gh, kw, T)
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    print("capture of a first call, T=24", flush=True)
    from mlsys26_flashinfer_moe_amd import moe
    saved = moe._workspaces
    moe._workspaces = moe.WorkspaceCache()      # no stream has a workspace yet
    try:
        with torch.cuda.graph(g):   # torch's own capture stream
            gh.pkg.run(**kw, output=out)
    finally:
        moe._workspaces, fresh = saved, moe._workspaces
    assert len(fresh._cache) == 1 and next(iter(fresh._cache.values())).captured
    for rep in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref), f"replay {rep} differs from the eager result"
        _ = (torch.randn(1 << 20, device=dev) * 2).sum().item()


def test_replay_after_a_larger_eager_call_on_the_capture_stream():
    """A graph captured at T=32 on stream s keeps its workspace when an eager call of T=700 on s
    needs a larger one: the replay still equals the T=32 eager result, and the T=700 call's
    result is unchanged by the replay."""
    from mlsys26_flashinfer_moe_amd import moe
    gh = _gh()
    dev = torch.device("cuda:0")
    w = gh.inputs.make_weights(4200, dev)
    s = torch.cuda.Stream(dev)
    small, big = _kw(gh, 32, 4201, w), _kw(gh, 700, 4202, w)
    saved = moe._workspaces
    moe._workspaces = moe.WorkspaceCache()      # a fresh cache: s (a pooled stream) has no workspace yet
    try:
        _capture_then_grow(gh, moe, dev, s, small, big)
    finally:
        moe._workspaces = saved


def _capture_then_grow(gh, moe, dev, s, small, big):
    ref_small = _eager_on(s, gh, small, 32)     # creates the T=32 workspace of s
    out = torch.empty((32, 7168), dtype=torch.bfloat16, device=dev)
    g = torch.cuda.CUDAGraph()
    torch.cuda.synchronize()
    print("capture at T=32, then an eager T=700 call on the same stream", flush=True)
    with torch.cuda.graph(g, stream=s):
        gh.pkg.run(**small, output=out)
    n_retired = len(moe._workspaces.retired)
    ref_big = _eager_on(s, gh, big, 700)        # replaces the workspace of s
    assert len(moe._workspaces.retired) == n_retired + 1, "the captured workspace was not retained"
    for rep in range(2):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(out, ref_small), f"replay {rep} differs from the eager result"
        again = _eager_on(s, gh, big, 700)
        assert torch.equal(again, ref_big)
