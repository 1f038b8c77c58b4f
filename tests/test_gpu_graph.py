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


@pytest.mark.parametrize("T", [48, 700])   # decode path (stream GEMMs) and tile path
def test_graph_replays_match_eager(T):
    gh = _gh()
    dev = torch.device("cuda:0")
    torch.manual_seed(T)
    w = gh.inputs.make_weights(31 + T, dev)
    logits, bias, hq, hs = gh.inputs.make_activations(T, 500 + T, dev)
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
