"""Benchmark of the MI355X fused FP8 MoE layer (routing through combine) on one GPU.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload t64] [--no-sweep] [--no-cpu]

A step is one call of the layer (routing, dispatch, GEMM1+SwiGLU+requant, GEMM2+combine) over
one batch of synthetic inputs already resident in HBM, through the C ABI as run() makes it: up
to 256 tokens moe_fp8_run_packed with the packed copy of the weight set that run()'s cache keeps
(built on the set's first call, outside the timed region; row_major_us_per_step times
moe_fp8_run on the row-major weights beside it), above 256 tokens moe_fp8_run. The headline
workload is the 64-token decode batch (H=7168, I=2048, 32 local of 256 experts, top-8);
`value` is its whole-layer algorithmic HBM throughput in GB/s:
    bytes = E_touched * 44,050,944 + T * 22,752 + 512
(per touched expert: W13 29,360,128 B + W2 14,680,064 B + their scales 10,752 B; per token:
hidden row 7,168 B + its 56 scales 224 B + router logits 1,024 B + bf16 output row 14,336 B;
the router bias 512 B), computed from the routing the step actually produced.
Three independent weight sets are rotated across steps so that every step streams its
weights from HBM (1.41 GB per set, far above the 256 MB last-level cache).

The JSON line also carries:
  roofline      the dominant kernel, GEMM1 (the one kernel of stage 2 of the layer: up to 64
                tokens gemm1_stream_dispatch_kernel<true> on the packed weights), timed with HIP
                events that the library records on the launch stream between the stages
                (moe_fp8_run_profiled);
  cpu_baseline  the numpy oracle (fp32 dequantise-and-matmul) on the same workload, timed on
                the host cores (median of 5 runs; the host's CPU model and count beside it);
  workloads     the same figures for the other four workloads (T=16, 1024 with offset 64,
                8192, 4096 skewed), each with the upstream activation quantiser
                (quantize_hidden: bf16 [T,7168] -> e4m3fn + scales [56,T]) timed beside the
                layer; its bytes are T * 21,728 (14,336 read, 7,168 + 224 written).
Per workload, us_per_step is the mean over the K timed C-ABI calls (one event pair around all
K); run_py_us_per_step the same through the Python entry point run() (argument checks,
workspace lookup and ctypes packing included; run_py_wall_us_per_step is its host wall
clock); us_median_call is the median of K calls timed one by one in a separate pass.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense OCP-fp8 MFMA
BYTES_PER_EXPERT = 44_050_944
BYTES_PER_TOKEN = 22_752
FLOPS_PER_ASSIGNMENT = 88_080_384    # 2*H*2I + 2*I*H
G1_BYTES_PER_EXPERT = 29_360_128 + 32 * 56 * 4
G2_BYTES_PER_EXPERT = 14_680_064 + 56 * 16 * 4
G1_FLOPS_PER_ASSIGNMENT = 2 * 7168 * 4096
G2_FLOPS_PER_ASSIGNMENT = 2 * 2048 * 7168


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="t64")
    ap.add_argument("--no-sweep", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--weight-sets", type=int, default=3)
    ap.add_argument("--copy-probe", action="store_true",
                    help="only run a plain 1 GiB device copy (calibration of rocprofv3 byte counters)")
    return ap.parse_args()


def routing_stats(ws, T):
    import torch
    torch.cuda.synchronize()
    cnt = ws.view("expert_count", torch.int32, 32).cpu()
    nloc = ws.view("token_nlocal", torch.int32, T).cpu()
    n = int(cnt.sum())
    e_touched = int((cnt > 0).sum())
    u = int((nloc > 0).sum())
    return n, e_touched, u


def workload_figures(T, n, e_touched, u, rows_per_item, requant_block=128):
    """Algorithmic work of the layer and of its GEMM1 kernel. GEMM1 reads the touched experts'
    W13 and block scales and each token's hidden row and scales once. Per assignment it writes,
    in the decode regime (items of <= 32 rows), the fp32 SwiGLU row (8,192 B), and up to 64
    tokens it reads the top-k lists (64 B per token) for the dispatch it rebuilds; on the tile
    path it writes the requantised fp8 row and its 2048 / requant_block scales (2,176 B with
    64-column blocks, 2,112 B with 128)."""
    layer_bytes = e_touched * BYTES_PER_EXPERT + T * BYTES_PER_TOKEN + 512
    layer_flops = n * FLOPS_PER_ASSIGNMENT
    g1_bytes = e_touched * G1_BYTES_PER_EXPERT + u * (7168 + 224)
    if rows_per_item <= 32:
        g1_bytes += n * 2048 * 4 + (T * 64 if rows_per_item == 16 else 0)
    else:
        g1_bytes += n * (2048 + (2048 // requant_block) * 4)
    return dict(layer_bytes=layer_bytes, layer_flops=layer_flops, g1_bytes=g1_bytes,
                g1_flops=n * G1_FLOPS_PER_ASSIGNMENT, g2_flops=n * G2_FLOPS_PER_ASSIGNMENT)


def gemm1_kernel_name(T, rows_per_item, packed=False):
    """The one kernel of stage 2 (GEMM1) of the layer for a batch of T tokens (packed: the
    packed copy of the weights, as run() streams it up to 256 tokens)."""
    if T <= 64:
        return (("gemm1_stream_dispatch_kernel<true>", "gemm1_stream_dispatch_packed") if packed else
                ("gemm1_stream_dispatch_kernel<false>", "gemm1_stream_dispatch"))
    if rows_per_item <= 32:
        return (f"gemm_stream_kernel<1, 2, {'true' if packed else 'false'}>",
                "gemm1_stream_packed" if packed else "gemm1_stream")
    return f"gemm_tile_kernel<true, {160 if rows_per_item > 128 else 128}>", "gemm1_tile"


def bench_workload(pkg, inputs, name, weight_sets, steps, warmup):
    import torch
    from mlsys26_flashinfer_moe_amd import _lib
    from mlsys26_flashinfer_moe_amd.moe import make_args, workspace_for

    dev = torch.device("cuda:0")
    wl = inputs.WORKLOADS[name]
    kw = inputs.make_workload(name, dev, weights=weight_sets[0])
    T = wl.num_tokens
    out = torch.empty((T, 7168), dtype=torch.bfloat16, device=dev)
    ws = workspace_for(T, dev)
    lib = _lib.load()
    stream = torch.cuda.current_stream(dev)
    sptr = stream.cuda_stream
    argsets = []
    for w in weight_sets:
        k2 = dict(kw)
        k2.update(gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3])
        argsets.append(make_args(k2["routing_logits"], k2["routing_bias"], k2["hidden_states"],
                                 k2["hidden_states_scale"], k2["gemm1_weights"], k2["gemm1_weights_scale"],
                                 k2["gemm2_weights"], k2["gemm2_weights_scale"], wl.local_expert_offset,
                                 inputs.ROUTED_SCALING_FACTOR, out))
    nbytes = ws.buffer.numel()
    R = len(argsets)
    # Up to 256 tokens run() streams a packed copy of each weight set, which its cache builds on
    # the first call with the set (outside every timed region here); the C-ABI steps do the same.
    packs = None
    if T <= _lib.PACKED_MAX_TOKENS:
        packs = [pkg.moe.packed_weights_for(w[0], w[2]) for w in weight_sets]
        if any(p is None for p in packs):
            packs = None
        torch.cuda.synchronize()
    npk = _lib.packed_weights_bytes()

    def step(i):
        if packs is not None:
            _lib.check(lib.moe_fp8_run_packed(argsets[i % R], packs[i % R].data_ptr(), npk, ws.ptr, nbytes, sptr),
                       "moe_fp8_run_packed")
        else:
            _lib.check(lib.moe_fp8_run(argsets[i % R], ws.ptr, nbytes, sptr), "moe_fp8_run")

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    n, e_touched, u = routing_stats(ws, T)

    # whole-layer timing through the C ABI: K steps between two synchronisations
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = ev0.elapsed_time(ev1) / steps
    row_major_ms = None
    if packs is not None:
        # the same K steps on the row-major weights (moe_fp8_run)
        ev0.record(stream)
        for i in range(steps):
            _lib.check(lib.moe_fp8_run(argsets[i % R], ws.ptr, nbytes, sptr), "moe_fp8_run")
        ev1.record(stream)
        torch.cuda.synchronize()
        row_major_ms = ev0.elapsed_time(ev1) / steps

    # the same K steps through the Python entry point run() (validation, workspace lookup and
    # argument packing included), host wall clock and HIP events
    kwsets = []
    for w in weight_sets:
        k2 = dict(kw)
        k2.update(gemm1_weights=w[0], gemm1_weights_scale=w[1], gemm2_weights=w[2], gemm2_weights_scale=w[3])
        kwsets.append(k2)
    for i in range(min(warmup, 3)):
        pkg.run(**kwsets[i % R], output=out)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ev0.record(stream)
    for i in range(steps):
        pkg.run(**kwsets[i % R], output=out)
    ev1.record(stream)
    torch.cuda.synchronize()
    run_wall = time.perf_counter() - t1
    run_ms = ev0.elapsed_time(ev1) / steps

    # per-call timing: an event before every call, for the median call duration
    pev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    for i in range(steps):
        pev[i].record(stream)
        step(i)
    pev[steps].record(stream)
    torch.cuda.synchronize()
    call_ms = sorted(pev[i].elapsed_time(pev[i + 1]) for i in range(steps))
    median_ms = call_ms[steps // 2] if steps % 2 else 0.5 * (call_ms[steps // 2 - 1] + call_ms[steps // 2])

    # stage timing of the same launches (moe_fp8_run_profiled): HIP events recorded by the
    # library on the launch stream between routing [+ dispatch], GEMM1 (one kernel) and
    # requantisation + GEMM2 + combine
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
    for e in evs:
        for x in e:
            x.record(stream)   # creates the underlying HIP event
    torch.cuda.synchronize()
    for i in range(steps):
        hev = (ctypes.c_void_p * 4)(*[x.cuda_event for x in evs[i]])
        pk = packs[i % R].data_ptr() if packs is not None else None
        _lib.check(lib.moe_fp8_run_profiled(argsets[i % R], pk, npk if pk else 0, ws.ptr, nbytes, sptr, hev),
                   "moe_fp8_run_profiled")
    torch.cuda.synchronize()
    stage_ms = [sum(evs[i][j].elapsed_time(evs[i][j + 1]) for i in range(steps)) / steps for j in range(3)]

    # the step before the layer: bf16 hidden states -> e4m3fn + 1x128 scales; three buffer
    # sets rotate so that large T streams from HBM
    qsets = []
    for i in range(3):
        x = torch.randn((T, 7168), device=dev, generator=torch.Generator(device=dev).manual_seed(40 + i))
        qsets.append((x.to(torch.bfloat16), torch.empty((T, 7168), dtype=torch.float8_e4m3fn, device=dev),
                      torch.empty((56, T), dtype=torch.float32, device=dev)))
    for i in range(3):
        pkg.quantize_hidden(qsets[i][0], qsets[i][1], qsets[i][2])
    q0, q1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    q0.record(stream)
    for i in range(steps):
        x, qo, so = qsets[i % 3]
        _lib.check(lib.moe_fp8_quantize_hidden(x.data_ptr(), _lib.HIDDEN_BF16, T, qo.data_ptr(), so.data_ptr(), sptr),
                   "moe_fp8_quantize_hidden")
    q1.record(stream)
    torch.cuda.synchronize()
    q_us = q0.elapsed_time(q1) / steps * 1e3
    q_bytes = T * (7168 * 2 + 7168 + 56 * 4)
    del qsets

    rpi = int(ws.layout.rows_per_item)
    f = workload_figures(T, n, e_touched, u, rpi, int(ws.layout.requant_block))
    us = ms_per_step * 1e3
    res = dict(T=T, offset=wl.local_expert_offset, assignments=n, experts_touched=e_touched,
               us_per_step=round(us, 2), us_median_call=round(median_ms * 1e3, 2),
               wall_us_per_step=round(wall / steps * 1e6, 2),
               run_py_us_per_step=round(run_ms * 1e3, 2), run_py_wall_us_per_step=round(run_wall / steps * 1e6, 2),
               hbm_gbs=round(f["layer_bytes"] / (us * 1e-6) / 1e9, 1),
               tflops=round(f["layer_flops"] / (us * 1e-6) / 1e12, 2),
               stage_us=dict(route_dispatch=round(stage_ms[0] * 1e3, 2), gemm1=round(stage_ms[1] * 1e3, 2),
                             requant_gemm2_combine=round(stage_ms[2] * 1e3, 2)))
    res["rows_per_item"] = rpi
    res["requant_block"] = int(ws.layout.requant_block)
    res["tokens_with_local"] = u
    res["gemm1_algorithmic_bytes"] = f["g1_bytes"]
    res["gemm1_algorithmic_flops"] = f["g1_flops"]
    if packs is not None:
        res["weights"] = "packed copy per weight set (as run() streams up to 256 tokens)"
        res["row_major_us_per_step"] = round(row_major_ms * 1e3, 2)
    res["hbm_roofline_frac"] = round(res["hbm_gbs"] / HBM_PEAK_GBS, 4)
    res["mfma_roofline_frac"] = round(res["tflops"] / FP8_PEAK_TFLOPS, 4)
    q_gbs = q_bytes / (q_us * 1e-6) / 1e9
    res["quantize_hidden"] = dict(us=round(q_us, 2), bytes=q_bytes, gbs=round(q_gbs, 1),
                                  hbm_roofline_frac=round(q_gbs / HBM_PEAK_GBS, 4))
    return res, f, stage_ms, kw


def cpu_baseline(kw, weight_set, reps=5):
    """The numpy oracle (definition mode) on the same workload, timed on this host."""
    import numpy as np
    import torch
    from oracle import layer as olayer
    try:
        from threadpoolctl import threadpool_info
        threads = max([p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"] or [1])
    except Exception:
        threads = 1
    u8 = lambda t: t.view(torch.uint8).cpu().numpy()
    args = (kw["routing_logits"].cpu().numpy(), kw["routing_bias"].float().cpu().numpy(),
            u8(kw["hidden_states"]), kw["hidden_states_scale"].cpu().numpy(), u8(weight_set[0]),
            weight_set[1].cpu().numpy(), u8(weight_set[2]), weight_set[3].cpu().numpy(),
            kw["local_expert_offset"], kw["routed_scaling_factor"])
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        r = olayer.layer_forward(*args, mode="definition")
        times.append(time.perf_counter() - t0)
    dt = float(np.median(times))
    T = args[0].shape[0]
    cnt = r["expert_count"]
    n, e_touched = int(cnt.sum()), int((cnt > 0).sum())
    b = e_touched * BYTES_PER_EXPERT + T * BYTES_PER_TOKEN + 512
    cpu_model = "unknown"
    try:
        with open("/proc/cpuinfo") as fh:
            cpu_model = next((l.split(":", 1)[1].strip() for l in fh if l.startswith("model name")), cpu_model)
    except OSError:
        pass
    return dict(value=round(b / dt / 1e9, 3), unit="GB/s", cores=int(threads), kind="port",
                cpu_model=cpu_model, host_cpus=os.cpu_count(),
                sample=f"whole layer, T={T}, {e_touched} touched experts, {n} assignments: median of "
                       f"{reps} runs of oracle.layer_forward(mode='definition'), {dt:.2f} s each, "
                       f"{sum(times):.1f} s in all (numpy: BLAS matmuls on {threads} threads, "
                       "element-wise work on 1)",
                seconds=round(dt, 3), us_per_step=round(dt * 1e6, 1))


def traffic_from_profiles(kernel_tag, workload):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc
    summary for this kernel and workload (FETCH_SIZE + WRITE_SIZE per dispatch, scaled by
    the counters' reading for a plain copy of known size), or None when there is none."""
    path = ROOT / "profiles" / f"{kernel_tag}_{workload}_traffic.json"
    if not path.exists():
        return None
    return json.loads(path.read_text()).get("hbm_bytes_per_launch")


def copy_probe():
    """A plain device-to-device copy of 1 GiB, five times: the reference point that scales
    rocprofv3's FETCH_SIZE / WRITE_SIZE readings to bytes."""
    import torch
    n = 1 << 30
    a = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes": n, "copies": 5}), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(this build runs the layer on a single MI355X).", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe:
        copy_probe()
        return
    import torch
    import __graft_entry__ as ge
    pkg = ge.load_package()
    from mlsys26_flashinfer_moe_amd import inputs

    dev = torch.device("cuda:0")
    weight_sets = [inputs.make_weights(777 + 13 * i, dev) for i in range(max(1, args.weight_sets))]
    torch.cuda.synchronize()

    names = [args.workload] + ([] if args.no_sweep else [n for n in inputs.WORKLOADS if n != args.workload])
    results = {}
    main_f = main_stage = main_kw = None
    for name in names:
        res, f, stage_ms, kw = bench_workload(pkg, inputs, name, weight_sets, args.steps, args.warmup)
        results[name] = res
        if name == args.workload:
            main_f, main_stage, main_kw = f, stage_ms, kw
        print(f"# {name}: {json.dumps(res)}", file=sys.stderr, flush=True)

    m = results[args.workload]
    T = m["T"]
    # Dominant kernel: GEMM1, the one kernel of stage 2 of moe_fp8_run (W13 is two thirds of the
    # weight bytes); HBM-bound up to T = 1024, MFMA-bound above. Its launch duration is the
    # HIP-event time of stage 2, recorded by the library on the launch stream.
    g1_ms = main_stage[1]
    rpi = m["rows_per_item"]
    kernel, tag = gemm1_kernel_name(T, rpi, "row_major_us_per_step" in m)
    if T <= 1024:
        roof = dict(kernel=kernel, bound="hbm", achieved=round(main_f["g1_bytes"] / (g1_ms * 1e-3) / 1e9, 1),
                    peak=HBM_PEAK_GBS, unit="GB/s")
    else:
        roof = dict(kernel=kernel, bound="mfma",
                    achieved=round(main_f["g1_flops"] / (g1_ms * 1e-3) / 1e12, 2), peak=FP8_PEAK_TFLOPS, unit="TFLOP/s")
    roof["frac"] = round(roof["achieved"] / roof["peak"], 4)
    roof["traffic"] = traffic_from_profiles(tag, args.workload)
    roof["avg_launch_us"] = round(g1_ms * 1e3, 2)
    roof["algorithmic_bytes"] = main_f["g1_bytes"]
    roof["algorithmic_flops"] = main_f["g1_flops"]

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(main_kw, weight_sets[0])

    line = {
        "metric": "MoE layer \u00b5s + fp8 TFLOPS / HBM GB/s vs roofline at T=64..8192, 1 GPU",
        "value": m["hbm_gbs"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m["us_per_step"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (fp32 accumulate)",
        "data": "synthetic: seeded N(0,1) activations, N(0,0.02) weights, fp8 block-quantised; "
                f"{args.weight_sets} weight sets rotated" + (
                    "; weights passed row-major, the layer streams the packed copy run() keeps per weight "
                    "set (built once per set, outside the timed region)" if "row_major_us_per_step" in m else ""),
        "config": {"workload": f"{args.workload}: T={T}, H=7168, I=2048, 32 local of 256 experts "
                               f"(offset {m['offset']}), top-8, 8 groups / top-4",
                   "global_batch": T, "seq_len": 1, "parallelism": "none (1 GPU)"},
        "us_per_step": m["us_per_step"],
        "tflops": m["tflops"],
        "hbm_roofline_frac": m["hbm_roofline_frac"],
        "roofline": roof,
        "cpu_baseline": cpu,
        "workloads": results,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
