"""GPU parity of the whole layer (routing through combine) against the CPU oracle.

Tolerances (bf16 output, compared as float32):
  vs the emulated oracle (same fp8 requantisation of the SwiGLU output as the kernels,
  1x128 blocks): |gpu - ref| <= 0.02 + 0.02 |ref| element-wise and relative RMS <= 0.01;
  the residual comes from fp32 summation order, which flips a few fp8 roundings of the
  intermediate (for constructed top-k lists the 0.02 grows as sqrt(max local experts per
  token / 2), since every local expert adds its own flips);
  vs the definition (fp32 intermediate, kernel.py's math without requantisation):
  |gpu - ref| <= 0.25 + 0.1 |ref| element-wise and relative RMS <= 0.05.
Sizes: T from 1 to 32768 (the largest puts parked GEMM2 rows beyond 2 GiB of the workspace).
The fp8 intermediate itself: its scales within 3e-4 relative, and at most 1 code step
apart on at most 1% of the bytes.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import layer as olayer
from oracle import routing as orouting

pytestmark = pytest.mark.gpu

TOPK = 8

_WEIGHTS = {}


def _gh():
    import gpu_helpers
    return gpu_helpers


def _weights():
    gh = _gh()
    if "w" not in _WEIGHTS:
        dev = torch.device("cuda:0")
        print("generating weights on cuda:0", flush=True)
        w = gh.inputs.make_weights(20240, dev)
        torch.cuda.synchronize()
        _WEIGHTS["w"] = w
        _WEIGHTS["np"] = tuple(t.view(torch.uint8).cpu().numpy() if t.dtype == torch.float8_e4m3fn
                               else t.cpu().numpy() for t in w)
    return _WEIGHTS["w"], _WEIGHTS["np"]


def _workload(name):
    gh = _gh()
    dev = torch.device("cuda:0")
    w, wnp = _weights()
    if name in ("t256", "t32768"):
        # t256: a decode batch between the named workloads (32-row items, separate
        # requantisation); t32768: a long prefill whose parked GEMM2 rows lie beyond 2 GiB of
        # the workspace (64-bit offsets in GEMM2 and the combine)
        T, seed = (256, 1005) if name == "t256" else (32768, 1006)
        logits, bias, hq, hs = gh.inputs.make_activations(T, seed, dev)
        kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
                  gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
                  local_expert_offset=0, routed_scaling_factor=gh.inputs.ROUTED_SCALING_FACTOR)
    else:
        kw = gh.inputs.make_workload(name, dev, weights=w)
    npkw = gh.to_numpy_inputs({**kw, "gemm1_weights": w[0][:1], "gemm2_weights": w[2][:1]})
    npkw["gemm1_weights"], npkw["gemm1_weights_scale"], npkw["gemm2_weights"], npkw["gemm2_weights_scale"] = wnp
    return kw, npkw


def _compare(got, ref, atol, rtol, rms_rel, what):
    err = np.abs(got - ref)
    bad = err > atol + rtol * np.abs(ref)
    rms = np.sqrt(np.mean((got - ref) ** 2)) / max(np.sqrt(np.mean(ref ** 2)), 1e-30)
    print(f"{what}: max err {err.max():.4g}, rel rms {rms:.4g}, violations {bad.sum()}", flush=True)
    assert not bad.any(), f"{what}: {bad.sum()} elements outside tolerance, max err {err.max():.4g}"
    assert rms <= rms_rel, f"{what}: relative RMS {rms:.4g} > {rms_rel}"


def _run_full(kw, out_dtype=torch.bfloat16):
    gh = _gh()
    T = kw["routing_logits"].shape[0]
    out = torch.full((T, 7168), float("nan"), dtype=out_dtype, device=kw["routing_logits"].device)
    gh.pkg.run(**kw, output=out)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("name,sample", [("t16", None), ("t64", None), ("t256", None), ("t1024_off64", None),
                                         ("t8192", 40), ("t4096_skew", 24), ("t32768", 24)])
def test_layer_matches_oracle(name, sample):
    kw, npkw = _workload(name)
    T = kw["routing_logits"].shape[0]
    print(f"layer {name} T={T}", flush=True)
    out = _run_full(kw)
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    tokens = None
    if sample is not None:
        rng = np.random.default_rng(T)
        tokens = np.sort(rng.choice(T, sample, replace=False))
    emu = olayer.layer_forward(**npkw, mode="emulated", tokens=tokens)
    sel = slice(None) if tokens is None else tokens
    _compare(got[sel], emu["output"], 0.02, 0.02, 0.01, f"{name} vs emulated oracle")
    ref = olayer.layer_forward(**npkw, mode="definition", tokens=tokens)
    _compare(got[sel], ref["output"], 0.25, 0.1, 0.05, f"{name} vs definition")
    # The fp8 requantisation of the SwiGLU output is the reference's own algorithm
    # (kernel.py:131-135, 64-column blocks); the layer must not be further from the fp32
    # definition than that algorithm is.
    ref64 = olayer.layer_forward(**npkw, mode="emulated", requant_block=64, tokens=tokens)
    rms = lambda x: float(np.sqrt(np.mean(np.square(x))))
    e_gpu = rms(got[sel] - ref["output"])
    e_ref = rms(ref64["output"] - ref["output"])
    print(f"{name}: rms(gpu - definition) {e_gpu:.4g}, rms(reference algorithm - definition) {e_ref:.4g}",
          flush=True)
    assert e_gpu <= 1.25 * e_ref
    # tokens with no local expert produce exact zeros
    zero = emu["token_nlocal"] == 0
    assert np.all(got[zero] == 0)
    if T > 9362:
        # parked rows (flat slot t*8 + k, 28,672 bytes each) of these tokens start beyond 2 GiB
        far = tokens[tokens * TOPK * 28672 >= 2 ** 31]
        assert np.any(emu["token_nlocal"][far] >= 2)


@pytest.mark.parametrize("T,offset", [(1, 0), (16, 0), (40, 224), (64, 0), (64, 96)])
def test_run_rebuilds_dispatch_in_gemm1(T, offset):
    """Up to 64 tokens moe_fp8_run launches routing alone, and every GEMM1 work-group rebuilds
    the dispatch in LDS; work-group 0 writes it to the workspace for the later kernels. That
    dispatch is bit-exact with the oracle's, and the output is bit-equal to the stage entry
    points' (routing and dispatch launched before GEMM1)."""
    gh = _gh()
    dev = torch.device("cuda:0")
    w, _ = _weights()
    print(f"run with dispatch in GEMM1: T={T} offset={offset}", flush=True)
    logits, bias, hq, hs = gh.inputs.make_activations(T, 3000 + T + offset, dev)
    rsf = gh.inputs.ROUTED_SCALING_FACTOR
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=offset, routed_scaling_factor=rsf)
    out = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
    ws = gh.new_workspace(T, dev)
    gh.run_layer(gh.make_args(**kw, output=out), ws)
    ids = gh.read(ws, "topk_ids", torch.int32, T * 8).reshape(T, 8)
    wts = gh.read(ws, "topk_weights", torch.float32, T * 8).reshape(T, 8)
    rid, rw = orouting.route(logits.cpu().numpy(), bias.float().cpu().numpy(), rsf)
    assert np.array_equal(ids, rid)
    assert np.array_equal(wts.view(np.uint32), rw.view(np.uint32))
    gh.check_dispatch(ws, rid, rw, offset, T)
    staged = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
    ws2 = gh.new_workspace(T, dev)
    args2 = gh.make_args(**kw, output=staged)
    gh.route_dispatch(args2, ws2)
    gh.gemm1(args2, ws2)
    gh.gemm2_combine(args2, ws2)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), staged.view(torch.int16))


@pytest.mark.parametrize("name", ["t64", "t256", "t1024_off64"])
def test_intermediate_fp8_matches_oracle(name):
    gh = _gh()
    kw, npkw = _workload(name)
    dev = kw["routing_logits"].device
    T = kw["routing_logits"].shape[0]
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    ws = gh.new_workspace(T, dev)
    args = gh.make_args(**kw, output=out)
    gh.route_dispatch(args, ws)
    gh.gemm1(args, ws)
    emu = olayer.layer_forward(**npkw, mode="emulated")
    n = len(emu["sorted_slot"])
    assert gh.counters(ws)[1] == n
    if ws.layout.rows_per_item <= 32:
        # decode regime: stage 2 leaves the fp32 SwiGLU rows, stage 3 requantises them.
        # GEMM1 outputs differ from the fp32 oracle by the MFMA's block-sum precision,
        # relative to the row's magnitude.
        c = gh.read(ws, "swiglu", torch.float32, n * 2048).reshape(n, 2048)
        ref = emu["swiglu"]
        row_max = np.max(np.abs(ref), axis=1, keepdims=True)
        err = np.abs(c - ref)
        bound = 1e-3 * np.abs(ref) + 2e-4 * row_max
        print(f"{name}: swiglu max err / bound {np.max(err / bound):.3f}", flush=True)
        assert np.all(err <= bound)
    gh.gemm2_combine(args, ws)
    act = gh.read(ws, "act", torch.uint8, n * 2048).reshape(n, 2048)
    sc = gh.read(ws, "act_scale", torch.float32, n * 16).reshape(n, 16)
    # The fp8 MFMA sums each 128-long K block at less than fp32 precision (observed
    # relative differences of the row maxima up to ~6e-5), so the scales agree to 3e-4.
    np.testing.assert_allclose(sc, emu["act_scale"], rtol=3e-4, atol=0)
    diff = act != emu["act"]
    print(f"{name}: act bytes differing {np.mean(diff):.4%}", flush=True)
    assert np.mean(diff) <= 0.01
    # Dequantised, the two intermediates differ by at most one fp8 step (12.5% of the
    # value) plus the accumulation difference, which is absolute: 4e-4 of the row maximum.
    deq_g = ofp8.decode(act) * np.repeat(sc, 128, axis=1)
    deq_r = ofp8.decode(emu["act"]) * np.repeat(emu["act_scale"], 128, axis=1)
    row_max = 448.0 * np.repeat(emu["act_scale"], 128, axis=1)
    err = np.abs(deq_g - deq_r)
    bound = 0.125 * np.abs(deq_r) + 4e-4 * row_max
    print(f"{name}: max err / bound {np.max(err / bound):.3f}", flush=True)
    assert np.all(err <= bound)


@pytest.mark.parametrize("name", ["t1024_off64", "t4096_skew"])
def test_tile_stage_repeated(name):
    """The GEMM1 tile kernel takes its units from per-XCD counters that the dispatch restarts.
    GEMM1 launched again after its result was wiped (no dispatch in between) redoes every unit:
    the launch before left the counters restarted. Staged and whole-layer runs agree bitwise."""
    gh = _gh()
    kw, _ = _workload(name)
    T = kw["routing_logits"].shape[0]
    print(f"tile stage repeated {name} T={T}", flush=True)
    whole = _run_full(kw)
    dev = kw["routing_logits"].device
    out = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
    ws = gh.new_workspace(T, dev)
    assert ws.layout.rows_per_item > 32
    args = gh.make_args(**kw, output=out)
    gh.route_dispatch(args, ws)
    gh.gemm1(args, ws)
    n = int(gh.counters(ws)[1])
    gh.write(ws, "act", np.zeros(n * 2048, dtype=np.uint8))
    gh.gemm1(args, ws)
    gh.gemm2_combine(args, ws)
    torch.cuda.synchronize()
    assert torch.equal(whole.view(torch.int16), out.view(torch.int16)), "staged and whole-layer runs differ"


def test_deterministic_and_fp32_output():
    kw, npkw = _workload("t1024_off64")
    a = _run_full(kw)
    b = _run_full(kw)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16)), "two runs differ bitwise"
    f = _run_full(kw, torch.float32)
    assert torch.equal(f.to(torch.bfloat16).view(torch.int16), a.view(torch.int16))


def test_cpu_output_and_inputs_are_moved():
    gh = _gh()
    kw, _ = _workload("t16")
    ref = _run_full(kw).cpu()
    cpu_kw = {k: (v.cpu() if isinstance(v, torch.Tensor) and v.numel() < 10_000_000 else v) for k, v in kw.items()}
    out = torch.empty((16, 7168), dtype=torch.bfloat16)
    gh.pkg.run(**cpu_kw, output=out)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def _given_topk(case, T, rng):
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    if case == "one_expert":                     # every token on local expert 5, nothing else local
        ids[:, 0] = 5
        ids[:, 1:] = np.where(ids[:, 1:] < 32, ids[:, 1:] + 32, ids[:, 1:])
    elif case == "none_local":
        ids = np.where(ids < 32, ids + 32, ids)
    elif case == "all_local":
        ids = np.stack([rng.permutation(32)[:8] for _ in range(T)]).astype(np.int32)
    elif case == "repeat":                       # a token naming one local expert twice
        ids[:, 0] = rng.integers(0, 32, size=T)
        ids[:, 1] = ids[:, 0]
    elif case == "few_local":
        # large-T items of every shape: expert 5 with 300 rows (two items), expert 17 with
        # exactly 160 (one full item), expert 9 with 200 (two), expert 30 with 20; tokens
        # 0..39 have two local experts (combined), tokens from 640 on none
        ids = np.where(ids < 32, ids + 32, ids)
        ids[0:300, 0] = 5
        ids[300:460, 0] = 9
        ids[460:480, 0] = 30
        ids[480:640, 0] = 17
        ids[0:40, 1] = 9
    w = (rng.random((T, 8)) * 0.5 + 0.1).astype(np.float32)
    return ids, w


@pytest.mark.parametrize("T,case", [(1, "all_local"), (40, "repeat"), (300, "all_local"),
                                    (513, "all_local"), (600, "one_expert"), (600, "none_local"),
                                    (4095, "all_local"), (4096, "all_local"), (4100, "few_local")])
def test_layer_edge_cases_given_topk(T, case):
    """The GEMM stages on constructed top-k lists: one token, a repeated expert, every token
    on one expert (many items of one expert on the tile path), nothing local, and at T >= 4096
    (items of up to 160 rows) items of every shape next to thousands of tokens without a
    local expert. T=513 is the first batch on the tile kernels; T=4095 and T=4096 put 1024 rows
    on every local expert, the largest batch of 128-row items and the first of 160-row items."""
    gh = _gh()
    dev = torch.device("cuda:0")
    w, wnp = _weights()
    print(f"layer edge case T={T} {case}", flush=True)
    rng = np.random.default_rng(T + len(case))
    ids, tw = _given_topk(case, T, rng)
    logits, bias, hq, hs = gh.inputs.make_activations(T, 77 + T, dev)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=0, routed_scaling_factor=2.5)
    out = torch.full((T, 7168), float("nan"), dtype=torch.bfloat16, device=dev)
    ws = gh.new_workspace(T, dev)
    gh.write(ws, "topk_ids", ids)
    gh.write(ws, "topk_weights", tw)
    args = gh.make_args(**kw, output=out)
    gh.route_dispatch(args, ws, skip_routing=1)
    gh.gemm1(args, ws)
    gh.gemm2_combine(args, ws)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    npkw = gh.to_numpy_inputs({**kw, "gemm1_weights": w[0][:1], "gemm2_weights": w[2][:1]})
    npkw["gemm1_weights"], npkw["gemm1_weights_scale"], npkw["gemm2_weights"], npkw["gemm2_weights_scale"] = wnp
    tokens = None if T <= 40 else np.sort(rng.choice(T, 24, replace=False))
    if case == "few_local":   # every kind of token: 2 local experts, each item's edges, none
        tokens = np.unique(np.concatenate([tokens, [0, 39, 40, 299, 300, 459, 460, 479, 480, 639, 640, T - 1]]))
    emu = olayer.layer_forward(**npkw, mode="emulated", topk=(ids, tw), tokens=tokens)
    sel = slice(None) if tokens is None else tokens
    if case == "none_local":
        assert np.all(got == 0)
        return
    # Each output element sums one contribution per local expert, and each carries the fp8
    # rounding flips of its intermediate; with up to 8 local experts per token the element-wise
    # bound grows with the square root of that count (the relative RMS bound does not).
    nloc = int(np.max(np.sum(ids[sel] < 32, axis=1)))
    atol = 0.02 * float(np.sqrt(max(1.0, nloc / 2.0)))
    _compare(got[sel], emu["output"], atol, 0.02, 0.01, f"T={T} {case} vs emulated oracle")
    if case == "few_local":
        assert ws.layout.rows_per_item == 160
        assert np.all(got[640:] == 0)


def test_layer_last_expert_group():
    """local_expert_offset = 224: the device owns the last routing group."""
    gh = _gh()
    dev = torch.device("cuda:0")
    w, wnp = _weights()
    T = 100
    logits, bias, hq, hs = gh.inputs.make_activations(T, 91, dev, local_expert_offset=224)
    kw = dict(routing_logits=logits, routing_bias=bias, hidden_states=hq, hidden_states_scale=hs,
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=224, routed_scaling_factor=2.5)
    print("layer offset 224 T=100", flush=True)
    got = _run_full(kw).float().cpu().numpy()
    npkw = gh.to_numpy_inputs({**kw, "gemm1_weights": w[0][:1], "gemm2_weights": w[2][:1]})
    npkw["gemm1_weights"], npkw["gemm1_weights_scale"], npkw["gemm2_weights"], npkw["gemm2_weights_scale"] = wnp
    emu = olayer.layer_forward(**npkw, mode="emulated")
    assert emu["token_nlocal"].sum() > 0
    _compare(got, emu["output"], 0.02, 0.02, 0.01, "offset 224 vs emulated oracle")


def test_zero_tokens():
    gh = _gh()
    dev = torch.device("cuda:0")
    w, _ = _weights()
    kw = dict(routing_logits=torch.zeros((0, 256), device=dev), routing_bias=torch.zeros(256, device=dev),
              hidden_states=torch.zeros((0, 7168), device=dev).to(torch.float8_e4m3fn),
              hidden_states_scale=torch.zeros((56, 0), device=dev),
              gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3],
              local_expert_offset=0, routed_scaling_factor=2.5)
    out = torch.empty((0, 7168), dtype=torch.bfloat16, device=dev)
    assert gh.pkg.run(**kw, output=out) is None
    torch.cuda.synchronize()
