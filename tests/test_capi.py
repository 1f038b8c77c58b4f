"""CPU-side checks of the C ABI: the library loads, exports every function declared in
include/moe_fp8.h, computes consistent workspace layouts, and rejects bad arguments
with the documented codes before touching the GPU."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def lib(pkg):
    return pkg._lib.load()


def test_exports_every_declared_function(pkg, lib):
    header = (ROOT / "include" / "moe_fp8.h").read_text()
    declared = set(re.findall(r"^\s*(?:int|size_t|const char\*)\s+(moe_fp8_\w+)\s*\(", header, re.M))
    assert declared == set(pkg._lib.EXPORTED_SYMBOLS)
    for name in declared:
        assert hasattr(lib, name), name


def test_constants_match_header(pkg):
    header = (ROOT / "include" / "moe_fp8.h").read_text()
    vals = dict(re.findall(r"#define\s+(MOE_FP8_\w+)\s+(-?\d+)\b", header))
    L = pkg._lib
    assert int(vals["MOE_FP8_HIDDEN"]) == L.HIDDEN and int(vals["MOE_FP8_INTER"]) == L.INTER
    assert int(vals["MOE_FP8_EXPERTS_LOCAL"]) == L.EXPERTS_LOCAL
    for name in ("OK", "EINVAL_POINTER", "EINVAL_TOKENS", "EWORKSPACE", "EINVAL_BIAS_DTYPE",
                 "EINVAL_OUT_DTYPE", "ELAUNCH", "EDEVICE", "EINVAL_HIDDEN_DTYPE", "ESTATIC_TOKENS", "EPACKED", "EALIGN",
                 "STATIC_MAX_TOKENS", "PACKED_MAX_TOKENS"):
        assert int(vals["MOE_FP8_" + name]) == getattr(L, name)
    for name in ("HIDDEN_F32", "HIDDEN_BF16", "HIDDEN_F16", "BIAS_F32", "BIAS_BF16", "BIAS_F16"):
        assert int(vals["MOE_FP8_" + name]) == getattr(L, name)


def test_struct_sizes(pkg):
    # 14 fields with natural alignment on x86-64
    assert ctypes.sizeof(pkg._lib.MoeFp8Args) == 104
    assert ctypes.sizeof(pkg._lib.MoeFp8Layout) == 18 * 8 + 8 * 4


@pytest.mark.parametrize("T", [0, 1, 15, 16, 17, 64, 257, 1024, 4096, 8192, 65536])
def test_layout_consistent(pkg, T):
    L = pkg._lib.workspace_layout(T)
    assert L.num_tokens == T and L.max_assignments == 8 * T
    assert L.route_blocks == (T + 15) // 16
    assert L.max_work_items == 32 + (8 * T + L.rows_per_item - 1) // L.rows_per_item
    assert L.counters == 0
    # up to 64 tokens (16-row items) GEMM2 combines in LDS (no parked rows); items of up to 32
    # rows (up to 256 tokens) keep GEMM1's fp32 SwiGLU rows; up to 128-row items (below 4096
    # tokens) requantise per 64 columns, the reference's block; the 160-row items per 128
    decode = L.rows_per_item == 16
    assert L.rows_per_item == (16 if T <= 64 else 32 if T <= 256 else L.rows_per_item)
    assert L.requant_block == (64 if L.rows_per_item <= 128 else 128)
    arrays = [
        ("topk_ids", 4 * 8 * T), ("topk_weights", 4 * 8 * T), ("expert_count", 4 * 32),
        ("expert_start", 4 * 33), ("sorted_token", 4 * 8 * T), ("sorted_weight", 4 * 8 * T),
        ("sorted_slot", 4 * 8 * T), ("token_nlocal", 4 * T), ("slot_rank", 4 * 8 * T),
        ("block_count", 4 * 32 * L.route_blocks), ("work_items", 16 * L.max_work_items),
        ("counters", 4 * 96), ("act", 8 * T * 2048), ("act_scale", 4 * 8 * T * 2048 // 64),
        ("partial", 0 if decode else 4 * 8 * T * 7168),
        ("swiglu", 4 * 8 * T * 2048 if L.rows_per_item <= 32 else 0), ("row_dest", 4 * 8 * T),
    ]
    spans = sorted((getattr(L, n), getattr(L, n) + b, n) for n, b in arrays)
    for (a0, a1, an), (b0, b1, bn) in zip(spans, spans[1:]):
        assert a1 <= b0, f"{an} overlaps {bn}"
    for off, _, n in spans:
        assert off % 256 == 0, n
    assert spans[-1][1] <= L.total_bytes
    assert pkg._lib.workspace_bytes(T) == L.total_bytes


def test_workspace_size_is_non_decreasing(pkg):
    """A workspace sized for T_max serves every T <= T_max, across the regime boundaries (16-row
    items up to 64 tokens, 32-row items up to 256, 128-row tiles below 4096, 160-row above)."""
    L = pkg._lib
    Ts = list(range(0, 70)) + list(range(250, 262)) + list(range(4088, 4100)) + [8192, 32768]
    sizes = [L.workspace_bytes(T) for T in Ts]
    assert all(a <= b for a, b in zip(sizes, sizes[1:])), [(T, s) for T, s in zip(Ts, sizes)]


def test_invalid_tokens(pkg, lib):
    assert lib.moe_fp8_workspace_bytes(-1) == 0
    assert lib.moe_fp8_workspace_bytes((1 << 20) + 1) == 0
    lay = pkg._lib.MoeFp8Layout()
    assert lib.moe_fp8_workspace_layout(-5, ctypes.byref(lay)) == pkg._lib.EINVAL_TOKENS


def _args(pkg, T=4):
    a = pkg._lib.MoeFp8Args()
    fake = 0x1000
    for f in ("routing_logits", "routing_bias", "hidden_states", "hidden_states_scale", "gemm1_weights",
              "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale", "output"):
        setattr(a, f, fake)
    a.num_tokens = T
    a.routed_scaling_factor = 2.5
    return a


def test_argument_errors_are_reported_before_any_launch(pkg, lib):
    L = pkg._lib
    big = L.workspace_bytes(4)
    a = _args(pkg)
    assert lib.moe_fp8_run(None, 0x1000, big, None) == L.EINVAL_POINTER
    a.hidden_states = None
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EINVAL_POINTER
    a = _args(pkg)
    a.routing_logits = None
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EINVAL_POINTER
    # ...but dispatch of given top-k lists does not need the router inputs (with a GPU present
    # these placeholder addresses would pass every check and be launched on: not tried there)
    import torch
    if not torch.cuda.is_available():
        assert lib.moe_fp8_route_dispatch(ctypes.byref(a), 1, 0x1000, big, None) == L.EDEVICE
    a = _args(pkg)
    a.num_tokens = -1
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EINVAL_TOKENS
    a = _args(pkg)
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big - 1, None) == L.EWORKSPACE
    assert lib.moe_fp8_run(ctypes.byref(a), None, big, None) == L.EWORKSPACE
    a.routing_bias_dtype = 3
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EINVAL_BIAS_DTYPE
    a = _args(pkg)
    a.output_dtype = 2
    assert lib.moe_fp8_gemm2_combine(ctypes.byref(a), 0x1000, big, None) == L.EINVAL_OUT_DTYPE
    # the evented variant: all four events are required, and argument errors come first
    a = _args(pkg)
    ev = (ctypes.c_void_p * 4)(0x10, 0x20, 0x30, 0x40)
    assert lib.moe_fp8_run_profiled(ctypes.byref(a), None, 0, 0x1000, big, None, None) == L.EINVAL_POINTER
    assert lib.moe_fp8_run_profiled(ctypes.byref(a), None, 0, 0x1000, big, None,
                                    (ctypes.c_void_p * 4)(0x10, 0x20, None, 0x40)) == L.EINVAL_POINTER
    assert lib.moe_fp8_run_profiled(ctypes.byref(a), None, 0, 0x1000, big - 1, None, ev) == L.EWORKSPACE
    assert lib.moe_fp8_run_profiled(ctypes.byref(a), 0x1000, 4096, 0x1000, big, None, ev) == L.EPACKED
    # T = 0 is a no-op that succeeds without a device
    a = _args(pkg, 0)
    assert lib.moe_fp8_run(ctypes.byref(a), None, 0, None) == L.OK
    for code in (0, -1, -2, -3, -4, -5, -6, -7, -8, -99):
        assert len(L.strerror(code)) > 5
    assert b"gfx950" in lib.moe_fp8_version()


def test_packed_weight_entry_points(pkg, lib):
    """The packed copy of W13 + W2 is exactly their size; missing or short buffers are reported
    before anything is launched (also without a GPU)."""
    L = pkg._lib
    n = L.packed_weights_bytes()
    assert n == 32 * 4096 * 7168 + 32 * 7168 * 2048 == 1_409_286_144
    a = _args(pkg)
    assert lib.moe_fp8_pack_weights(None, 0x1000, n, None) == L.EINVAL_POINTER
    a.gemm2_weights = None
    assert lib.moe_fp8_pack_weights(ctypes.byref(a), 0x1000, n, None) == L.EINVAL_POINTER
    a = _args(pkg)
    assert lib.moe_fp8_pack_weights(ctypes.byref(a), None, n, None) == L.EPACKED
    assert lib.moe_fp8_pack_weights(ctypes.byref(a), 0x1000, n - 1, None) == L.EPACKED
    big = L.workspace_bytes(4)
    assert lib.moe_fp8_run_packed(ctypes.byref(a), None, n, 0x1000, big, None) == L.EPACKED
    assert lib.moe_fp8_run_packed(ctypes.byref(a), 0x1000, n - 1, 0x1000, big, None) == L.EPACKED
    # then the checks of moe_fp8_run
    assert lib.moe_fp8_run_packed(ctypes.byref(a), 0x1000, n, 0x1000, big - 1, None) == L.EWORKSPACE
    a.num_tokens = -1
    assert lib.moe_fp8_run_packed(ctypes.byref(a), 0x1000, n, 0x1000, big, None) == L.EINVAL_TOKENS
    assert len(L.strerror(L.EPACKED)) > 5


def test_no_device_is_reported(pkg, lib):
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    L = pkg._lib
    a = _args(pkg)
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, L.workspace_bytes(4), None) == L.EDEVICE


@pytest.mark.parametrize("field,offset", [
    ("routing_logits", 8), ("routing_bias", 2), ("hidden_states", 8), ("hidden_states_scale", 2),
    ("gemm1_weights", 8), ("gemm1_weights_scale", 2), ("gemm2_weights", 8), ("gemm2_weights_scale", 2),
    ("output", 4)])
def test_misaligned_pointers_are_reported(pkg, lib, field, offset):
    """A pointer off the alignment of the kernels' widest access to it is MOE_FP8_EALIGN, before
    anything is launched. Calls whose placeholder addresses would pass every check are made only
    without a GPU (they then stop at EDEVICE)."""
    import torch
    L = pkg._lib
    big = L.workspace_bytes(4)
    a = _args(pkg)
    setattr(a, field, 0x1000 + offset)
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EALIGN
    assert lib.moe_fp8_run_static(ctypes.byref(a), None) == L.EALIGN
    if field not in ("routing_logits", "routing_bias"):
        assert lib.moe_fp8_gemm1(ctypes.byref(a), 0x1000, big, None) == L.EALIGN
    elif not torch.cuda.is_available():
        # the GEMM stages do not read the router inputs and do not check them
        assert lib.moe_fp8_gemm1(ctypes.byref(a), 0x1000, big, None) == L.EDEVICE
    if not torch.cuda.is_available():
        # bf16 bias (2 bytes) and bf16 output (8) accept what fp32 would not
        a = _args(pkg)
        a.routing_bias = 0x1002
        a.routing_bias_dtype = L.BIAS_BF16
        a.output = 0x1008
        a.output_dtype = L.OUT_BF16
        assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EDEVICE
        a.routing_bias_dtype = L.BIAS_F32
        assert lib.moe_fp8_run(ctypes.byref(a), 0x1000, big, None) == L.EALIGN


def test_misaligned_workspace_and_buffers_are_reported(pkg, lib):
    L = pkg._lib
    big = L.workspace_bytes(4)
    a = _args(pkg)
    assert lib.moe_fp8_run(ctypes.byref(a), 0x1080, big, None) == L.EALIGN
    assert lib.moe_fp8_workspace_init(0x1080, big, None) == L.EALIGN
    n = L.packed_weights_bytes()
    assert lib.moe_fp8_run_packed(ctypes.byref(a), 0x1008, n, 0x1000, big, None) == L.EALIGN
    assert lib.moe_fp8_pack_weights(ctypes.byref(a), 0x1008, n, None) == L.EALIGN
    a.gemm2_weights = 0x2004
    assert lib.moe_fp8_pack_weights(ctypes.byref(a), 0x1000, n, None) == L.EALIGN
    f = lib.moe_fp8_quantize_hidden
    assert f(0x1008, L.HIDDEN_BF16, 4, 0x2000, 0x3000, None) == L.EALIGN
    assert f(0x1000, L.HIDDEN_BF16, 4, 0x2004, 0x3000, None) == L.EALIGN
    assert f(0x1000, L.HIDDEN_BF16, 4, 0x2000, 0x3002, None) == L.EALIGN
    assert "aligned" in L.strerror(L.EALIGN)


def test_quantize_hidden_argument_errors(pkg, lib):
    L = pkg._lib
    f = lib.moe_fp8_quantize_hidden
    assert f(0x1000, L.HIDDEN_BF16, -1, 0x2000, 0x3000, None) == L.EINVAL_TOKENS
    assert f(0x1000, L.HIDDEN_BF16, (1 << 20) + 1, 0x2000, 0x3000, None) == L.EINVAL_TOKENS
    assert f(None, L.HIDDEN_BF16, 4, 0x2000, 0x3000, None) == L.EINVAL_POINTER
    assert f(0x1000, L.HIDDEN_BF16, 4, None, 0x3000, None) == L.EINVAL_POINTER
    assert f(0x1000, L.HIDDEN_BF16, 4, 0x2000, None, None) == L.EINVAL_POINTER
    assert f(0x1000, 3, 4, 0x2000, 0x3000, None) == L.EINVAL_HIDDEN_DTYPE
    assert f(None, 3, 0, None, None, None) == L.OK   # T = 0: nothing to do
    import torch
    if not torch.cuda.is_available():
        assert f(0x1000, L.HIDDEN_BF16, 4, 0x2000, 0x3000, None) == L.EDEVICE


def test_static_entry_reports_argument_errors_first(pkg, lib):
    """moe_fp8_run_static checks every argument before its first call on a device queues the
    clear kernel of its built-in workspace: null pointers, bad dtypes and oversize batches come
    back as their codes with no device at hand (the GPU tests cover the device path)."""
    L = pkg._lib
    f = lib.moe_fp8_run_static
    assert f(None, None) == L.EINVAL_POINTER
    a = _args(pkg)
    a.gemm2_weights_scale = None
    assert f(ctypes.byref(a), None) == L.EINVAL_POINTER
    a = _args(pkg)
    a.routing_logits = None
    assert f(ctypes.byref(a), None) == L.EINVAL_POINTER
    a = _args(pkg)
    a.routing_bias_dtype = 7
    assert f(ctypes.byref(a), None) == L.EINVAL_BIAS_DTYPE
    a = _args(pkg)
    a.output_dtype = 5
    assert f(ctypes.byref(a), None) == L.EINVAL_OUT_DTYPE
    a = _args(pkg, L.STATIC_MAX_TOKENS + 1)
    assert f(ctypes.byref(a), None) == L.ESTATIC_TOKENS
    a = _args(pkg, -2)
    assert f(ctypes.byref(a), None) == L.EINVAL_TOKENS
    assert f(ctypes.byref(_args(pkg, 0)), None) == L.OK
    import torch
    if not torch.cuda.is_available():
        assert f(ctypes.byref(_args(pkg)), None) == L.EDEVICE
