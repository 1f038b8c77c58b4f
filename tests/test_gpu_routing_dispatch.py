"""GPU parity of routing + dispatch (moe_fp8_route_dispatch) against the oracle.

Up to 256 tokens a wavefront routes one token (route_wide_kernel); above, sixteen lanes route one
token (route_kernel, which also ranks the slots for the multi-work-group dispatch). Both are
checked on the golden router logits, every bias dtype, ties and extreme values.

Bar: bit-exact. Expert ids, routing weights (as fp32 bit patterns), histogram, CSR
offsets, the stable bucket permutation, per-token local counts and the GEMM work list
must equal the oracle's exactly.
"""
import numpy as np
import pytest
import torch

from oracle import routing as orouting

pytestmark = pytest.mark.gpu

from pathlib import Path  # noqa: E402

GOLD = np.load(Path(__file__).parent / "golden" / "routing_golden.npz")


def _gh():
    import gpu_helpers
    return gpu_helpers


def _route_gpu(logits_np, bias_np, offset=0, rsf=2.5, bias_dtype=torch.float32):
    gh = _gh()
    dev = torch.device("cuda:0")
    T = logits_np.shape[0]
    logits = torch.from_numpy(np.ascontiguousarray(logits_np)).to(dev)
    bias = torch.from_numpy(np.ascontiguousarray(bias_np)).to(bias_dtype).to(dev)
    ws = gh.new_workspace(T, dev)
    args = gh.routing_args(logits, bias, offset, rsf)
    print(f"route_dispatch T={T} offset={offset} bias={bias_dtype}", flush=True)
    gh.route_dispatch(args, ws)
    return ws, gh


@pytest.mark.parametrize("part", [0, 1, 2])
def test_routing_bit_exact_on_golden_logits(part):
    m = GOLD["bias_index"] == part
    logits, bias = GOLD["logits"][m], GOLD["bias_sets"][part]
    ws, gh = _route_gpu(logits, bias)
    T = logits.shape[0]
    ids = gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8)
    w = gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8)
    rid, rw = orouting.route(logits, bias, 2.5)
    assert np.array_equal(ids, rid)
    assert np.array_equal(w.view(np.uint32), rw.view(np.uint32))
    # and the independent router's expert sets
    assert np.array_equal(np.sort(ids, axis=1), GOLD["ids_sorted"][m])
    gh.check_dispatch(ws, rid, rw, 0, T)


@pytest.mark.parametrize("part", [0, 1, 2])
def test_routing_bit_exact_on_golden_logits_large_batches(part):
    """Above 256 tokens sixteen lanes route a token (route_kernel): the golden rows of each bias
    set repeated to 3x their count."""
    m = GOLD["bias_index"] == part
    logits, bias = np.concatenate([GOLD["logits"][m]] * 3), GOLD["bias_sets"][part]
    T = logits.shape[0]
    assert T > 256
    ws, gh = _route_gpu(logits, bias)
    rid, rw = orouting.route(logits, bias, 2.5)
    assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
    assert np.array_equal(gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8).view(np.uint32),
                          rw.view(np.uint32))
    gh.check_dispatch(ws, rid, rw, 0, T)


@pytest.mark.parametrize("part", [0, 1, 2])
def test_routing_bit_exact_on_golden_logits_small_batches(part):
    """Up to 256 tokens a wavefront routes one token (route_wide_kernel): the golden rows of each
    bias set in batches of 64 and of 1."""
    m = GOLD["bias_index"] == part
    logits_all, bias = GOLD["logits"][m], GOLD["bias_sets"][part]
    for lo in range(0, logits_all.shape[0], 64):
        logits = logits_all[lo:lo + 64]
        for batch in ((logits,) if lo else (logits, logits[:1])):
            ws, gh = _route_gpu(batch, bias)
            T = batch.shape[0]
            rid, rw = orouting.route(batch, bias, 2.5)
            assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
            assert np.array_equal(gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8).view(np.uint32),
                                  rw.view(np.uint32))


@pytest.mark.parametrize("T", [40, 77, 300])
@pytest.mark.parametrize("bias_dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_routing_bias_dtypes(bias_dtype, T):
    rng = np.random.default_rng(21)
    logits = rng.standard_normal((T, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    ws, gh = _route_gpu(logits, bias, bias_dtype=bias_dtype)
    bias_cast = torch.from_numpy(bias).to(bias_dtype).float().numpy()
    rid, rw = orouting.route(logits, bias_cast, 2.5)
    assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
    assert np.array_equal(gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8).view(np.uint32),
                          rw.view(np.uint32))


@pytest.mark.parametrize("repeat", [1, 50])
def test_routing_ties_and_extremes(repeat):
    """Six special rows (T = 6: route_wide_kernel), and the same rows 50 times (T = 300: route_kernel)."""
    T = 6
    logits = np.zeros((T, 256), np.float32)
    logits[1] = 100.0                       # saturated sigmoid: all ties at 1.0
    logits[2] = -100.0                      # saturated low
    logits[3, ::7] = np.inf
    logits[4, 5] = 1e30
    logits[5] = np.linspace(-50, 50, 256, dtype=np.float32)
    bias = np.zeros(256, np.float32)
    bias[200] = -np.inf                     # an expert that can never win unless forced
    logits = np.concatenate([logits] * repeat)
    T = logits.shape[0]
    ws, gh = _route_gpu(logits, bias, rsf=1.0)
    rid, rw = orouting.route(logits, bias, 1.0)
    assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
    assert np.array_equal(gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8).view(np.uint32),
                          rw.view(np.uint32))


@pytest.mark.parametrize("T,offset", [(1, 0), (5, 224), (16, 0), (17, 64), (64, 0), (255, 32),
                                      (256, 0), (257, 0), (1000, 250), (4096, 0), (8192, 96), (3, -3),
                                      (16384, 0), (16385, 32), (65536, 96)])
def test_dispatch_matches_oracle(T, offset):
    """Above 16384 tokens (1024 routing work-groups) the per-work-group prefixes come from
    block_scan_kernel instead of every placing work-group's own reduction."""
    rng = np.random.default_rng(T * 7 + offset + 1000)
    logits = rng.standard_normal((T, 256)).astype(np.float32)
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    ws, gh = _route_gpu(logits, bias, offset=offset)
    rid, rw = orouting.route(logits, bias, 2.5)
    assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
    gh.check_dispatch(ws, rid, rw, offset, T)


@pytest.mark.parametrize("T", [60, 300])
@pytest.mark.parametrize("case", ["one_expert", "none_local", "all_local", "repeat"])
def test_dispatch_given_topk(case, T):
    gh = _gh()
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(4)
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    if case == "one_expert":
        ids[:, 0] = 5                                   # every token on local expert 5
        ids[:, 1:] = np.where(ids[:, 1:] < 32, ids[:, 1:] + 32, ids[:, 1:])
        ids[:, 1:] = np.where(ids[:, 1:] == 5, 40, ids[:, 1:])
    elif case == "none_local":
        ids = np.where(ids < 32, ids + 32, ids)
    elif case == "all_local":
        ids = np.stack([rng.permutation(32)[:8] for _ in range(T)]).astype(np.int32)
    elif case == "repeat":
        ids[:, 1] = ids[:, 0]                           # a token naming one expert twice
    w = rng.random((T, 8)).astype(np.float32)
    ws = gh.new_workspace(T, dev)
    gh.write(ws, "topk_ids", ids)
    gh.write(ws, "topk_weights", w)
    logits = torch.zeros((T, 256), device=dev)
    args = gh.routing_args(logits, torch.zeros(256, device=dev), 0, 1.0)
    print(f"dispatch given top-k case={case}", flush=True)
    gh.route_dispatch(args, ws, skip_routing=1)
    gh.check_dispatch(ws, ids, w, 0, T)
    # the given lists are left untouched
    assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), ids)


def test_workspace_reuse_across_calls():
    """One workspace, successive calls with different T on one stream."""
    gh = _gh()
    dev = torch.device("cuda:0")
    ws = gh.new_workspace(2048, dev)
    for T, off in ((2048, 0), (40, 64), (700, 0), (2048, 32)):
        rng = np.random.default_rng(T + off)
        logits = rng.standard_normal((T, 256)).astype(np.float32)
        bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
        lt = torch.from_numpy(logits).to(dev)
        bt = torch.from_numpy(bias).to(dev)
        ws.layout = gh._lib.workspace_layout(T)
        args = gh.routing_args(lt, bt, off, 2.5)
        gh.route_dispatch(args, ws)
        rid, rw = orouting.route(logits, bias, 2.5)
        gh.check_dispatch(ws, rid, rw, off, T)


FEW_FINITE = {
    0: [],
    1: [77],
    5: [3, 17, 40, 70, 100],
    7: [0, 1, 2, 33, 34, 64, 96],
    "mixed": [0, 1, 32, 64, 96, 128, 129, 160, 192, 193, 224],
}


@pytest.mark.parametrize("T", [37, 300])
@pytest.mark.parametrize("case", list(FEW_FINITE))
def test_routing_fewer_than_top_k_finite_candidates(case, T):
    """Biases of -inf leave 0, 1, 5 or 7 finite biased scores in the kept groups (and 7 in a
    mix of finite and -inf group scores). As in kernel.py:522-534, the remaining top-k slots
    all name expert 0 (the first index of the -inf maximum, a chosen expert included), and the
    weights count each repeat. T=37 runs route_wide_kernel, T=300 route_kernel; both bias
    dtypes that can hold -inf in storage of their own are used (fp32, bf16)."""
    rng = np.random.default_rng(57 + T)
    logits = rng.standard_normal((T, 256)).astype(np.float32)
    bias = np.full(256, -np.inf, np.float32)
    fin = FEW_FINITE[case]
    bias[fin] = (rng.standard_normal(len(fin)) * 0.1).astype(np.float32)
    for bias_dtype in (torch.float32, torch.bfloat16):
        ws, gh = _route_gpu(logits, bias, offset=0, bias_dtype=bias_dtype)
        bias_cast = torch.from_numpy(bias).to(bias_dtype).float().numpy()
        rid, rw = orouting.route(logits, bias_cast, 2.5)
        assert np.all(rid[:, -1] == 0), "the last slot repeats expert 0"
        assert np.array_equal(gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8), rid)
        assert np.array_equal(gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8).view(np.uint32),
                              rw.view(np.uint32))
        gh.check_dispatch(ws, rid, rw, 0, T)
