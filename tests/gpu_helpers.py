"""Helpers for the GPU parity tests: run the C-ABI stages and read the workspace."""
from __future__ import annotations

import numpy as np
import torch

import __graft_entry__ as ge
from oracle import dispatch as odsp

pkg = ge.load_package()
from mlsys26_flashinfer_moe_amd import _lib, inputs  # noqa: E402
from mlsys26_flashinfer_moe_amd.moe import Workspace, make_args  # noqa: E402

DUMMY = {}


def dummy(dev):
    """Tiny non-null device buffers standing in for inputs a stage does not read."""
    if dev not in DUMMY:
        DUMMY[dev] = dict(
            hidden=torch.zeros((1, 16), dtype=torch.float8_e4m3fn, device=dev),
            scale=torch.zeros(16, dtype=torch.float32, device=dev),
            out=torch.zeros(16, dtype=torch.bfloat16, device=dev),
        )
    return DUMMY[dev]


def routing_args(logits: torch.Tensor, bias: torch.Tensor, offset: int, rsf: float, hidden=None):
    d = dummy(logits.device)
    T = logits.shape[0]
    h = hidden if hidden is not None else d["hidden"]
    a = make_args(logits, bias, h, d["scale"], d["hidden"], d["scale"], d["hidden"], d["scale"],
                  offset, rsf, d["out"])
    a.num_tokens = T
    return a


def new_workspace(T: int, dev) -> Workspace:
    return Workspace(T, dev)


def stream():
    return torch.cuda.current_stream().cuda_stream


def route_dispatch(args, ws: Workspace, skip_routing: int = 0):
    _lib.check(_lib.load().moe_fp8_route_dispatch(args, int(skip_routing), ws.ptr, ws.buffer.numel(), stream()),
               "moe_fp8_route_dispatch")


def gemm1(args, ws: Workspace):
    _lib.check(_lib.load().moe_fp8_gemm1(args, ws.ptr, ws.buffer.numel(), stream()), "moe_fp8_gemm1")


def gemm2_combine(args, ws: Workspace):
    _lib.check(_lib.load().moe_fp8_gemm2_combine(args, ws.ptr, ws.buffer.numel(), stream()),
               "moe_fp8_gemm2_combine")


def run_layer(args, ws: Workspace):
    _lib.check(_lib.load().moe_fp8_run(args, ws.ptr, ws.buffer.numel(), stream()), "moe_fp8_run")


def read(ws: Workspace, name: str, dtype: torch.dtype, count: int) -> np.ndarray:
    torch.cuda.synchronize()
    t = ws.view(name, dtype, count).cpu()
    if dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return t.numpy().copy()


def write(ws: Workspace, name: str, arr: np.ndarray):
    src = torch.from_numpy(np.ascontiguousarray(arr))
    ws.view(name, src.dtype, src.numel()).copy_(src.reshape(-1).to(ws.buffer.device))
    torch.cuda.synchronize()


def counters(ws: Workspace) -> np.ndarray:
    return read(ws, "counters", torch.int32, 16)


def to_numpy_inputs(kw: dict) -> dict:
    """run() keyword arguments on the GPU -> the oracle's numpy arguments."""
    u8 = lambda t: t.view(torch.uint8).cpu().numpy()
    return dict(
        routing_logits=kw["routing_logits"].cpu().numpy(),
        routing_bias=kw["routing_bias"].float().cpu().numpy(),
        hidden_states=u8(kw["hidden_states"]),
        hidden_states_scale=kw["hidden_states_scale"].cpu().numpy(),
        gemm1_weights=u8(kw["gemm1_weights"]),
        gemm1_weights_scale=kw["gemm1_weights_scale"].cpu().numpy(),
        gemm2_weights=u8(kw["gemm2_weights"]),
        gemm2_weights_scale=kw["gemm2_weights_scale"].cpu().numpy(),
        local_expert_offset=kw["local_expert_offset"],
        routed_scaling_factor=kw["routed_scaling_factor"],
    )


def check_dispatch(ws: Workspace, ids: np.ndarray, w: np.ndarray, offset: int, T: int):
    """The workspace's dispatch arrays are bit-exact with the oracle's dispatch of (ids, w)."""
    d = odsp.dispatch(ids, w, offset)
    n = int(d["expert_start"][-1])
    c = counters(ws)
    assert c[1] == n
    assert np.array_equal(read(ws, "expert_count", torch.int32, 32), d["expert_count"])
    assert np.array_equal(read(ws, "expert_start", torch.int32, 33), d["expert_start"])
    assert np.array_equal(read(ws, "sorted_slot", torch.int32, n), d["sorted_slot"])
    assert np.array_equal(read(ws, "sorted_token", torch.int32, n), d["sorted_token"])
    assert np.array_equal(read(ws, "sorted_weight", torch.float32, n).view(np.uint32),
                          d["sorted_weight"].view(np.uint32))
    assert np.array_equal(read(ws, "token_nlocal", torch.int32, T), d["token_nlocal"])
    if T > 256:
        # the multi-work-group dispatch also leaves GEMM2's destination of every bucket row: the
        # token if it has one local assignment, else -1 - the row's flat slot
        st, ss = d["sorted_token"], d["sorted_slot"]
        want = np.where(d["token_nlocal"][st] == 1, st, -1 - ss).astype(np.int32)
        assert np.array_equal(read(ws, "row_dest", torch.int32, n), want)
    rpi = int(ws.layout.rows_per_item)
    items = odsp.work_items(d["expert_count"], d["expert_start"], rpi)
    assert c[0] == len(items)
    got = read(ws, "work_items", torch.int32, 4 * len(items)).reshape(-1, 4)
    assert np.array_equal(got, items)
    # every bucket row is covered exactly once by the work list
    cover = np.zeros(n, dtype=np.int32)
    for e, r0, rows, _ in items:
        assert d["expert_start"][e] <= r0 and r0 + rows <= d["expert_start"][e + 1] and 0 < rows <= rpi
        cover[r0:r0 + rows] += 1
    assert np.all(cover == 1)
