"""ctypes binding of libmoe_fp8.so, the C ABI declared in include/moe_fp8.h.

This is the only place where Python touches the native library. There is no fallback:
if the shared library is missing or was built for another architecture, loading fails
with a RuntimeError naming the build step.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
LIB_PATH = PKG_DIR / "libmoe_fp8.so"

HIDDEN = 7168
INTER = 2048
EXPERTS_GLOBAL = 256
EXPERTS_LOCAL = 32
TOP_K = 8
N_GROUP = 8
TOPK_GROUP = 4
BLOCK = 128
H_BLOCKS = HIDDEN // BLOCK
I_BLOCKS = INTER // BLOCK
G1_BLOCKS = 2 * INTER // BLOCK
MAX_TOKENS = 1 << 20

BIAS_F32, BIAS_BF16, BIAS_F16 = 0, 1, 2
HIDDEN_F32, HIDDEN_BF16, HIDDEN_F16 = 0, 1, 2
OUT_BF16, OUT_F32 = 0, 1

OK = 0
EINVAL_POINTER = -1
EINVAL_TOKENS = -2
EWORKSPACE = -3
EINVAL_BIAS_DTYPE = -4
EINVAL_OUT_DTYPE = -5
ELAUNCH = -6
EDEVICE = -7
EINVAL_HIDDEN_DTYPE = -8
ESTATIC_TOKENS = -9
EPACKED = -10
EALIGN = -11
STATIC_MAX_TOKENS = 64
PACKED_MAX_TOKENS = 256
STATIC_SCRATCH_BYTES = 6 << 20

EXPORTED_SYMBOLS = (
    "moe_fp8_workspace_bytes",
    "moe_fp8_workspace_layout",
    "moe_fp8_workspace_init",
    "moe_fp8_run",
    "moe_fp8_run_profiled",
    "moe_fp8_run_static",
    "moe_fp8_packed_weights_bytes",
    "moe_fp8_pack_weights",
    "moe_fp8_run_packed",
    "moe_fp8_route_dispatch",
    "moe_fp8_gemm1",
    "moe_fp8_gemm2_combine",
    "moe_fp8_quantize_hidden",
    "moe_fp8_strerror",
    "moe_fp8_version",
)


class MoeFp8Args(ctypes.Structure):
    """struct moe_fp8_args."""

    _fields_ = [
        ("routing_logits", ctypes.c_void_p),
        ("routing_bias", ctypes.c_void_p),
        ("routing_bias_dtype", ctypes.c_int32),
        ("hidden_states", ctypes.c_void_p),
        ("hidden_states_scale", ctypes.c_void_p),
        ("gemm1_weights", ctypes.c_void_p),
        ("gemm1_weights_scale", ctypes.c_void_p),
        ("gemm2_weights", ctypes.c_void_p),
        ("gemm2_weights_scale", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int32),
        ("local_expert_offset", ctypes.c_int32),
        ("routed_scaling_factor", ctypes.c_float),
        ("output", ctypes.c_void_p),
        ("output_dtype", ctypes.c_int32),
    ]


class MoeFp8Layout(ctypes.Structure):
    """struct moe_fp8_layout: byte offsets of the workspace arrays."""

    _fields_ = [
        ("total_bytes", ctypes.c_size_t),
        ("topk_ids", ctypes.c_size_t),
        ("topk_weights", ctypes.c_size_t),
        ("expert_count", ctypes.c_size_t),
        ("expert_start", ctypes.c_size_t),
        ("sorted_token", ctypes.c_size_t),
        ("sorted_weight", ctypes.c_size_t),
        ("sorted_slot", ctypes.c_size_t),
        ("token_nlocal", ctypes.c_size_t),
        ("slot_rank", ctypes.c_size_t),
        ("block_count", ctypes.c_size_t),
        ("work_items", ctypes.c_size_t),
        ("counters", ctypes.c_size_t),
        ("act", ctypes.c_size_t),
        ("act_scale", ctypes.c_size_t),
        ("partial", ctypes.c_size_t),
        ("swiglu", ctypes.c_size_t),
        ("row_dest", ctypes.c_size_t),
        ("num_tokens", ctypes.c_int32),
        ("max_assignments", ctypes.c_int32),
        ("max_work_items", ctypes.c_int32),
        ("route_blocks", ctypes.c_int32),
        ("rows_per_item", ctypes.c_int32),
        ("requant_block", ctypes.c_int32),
        ("reserved", ctypes.c_int32 * 2),
    ]


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Loads libmoe_fp8.so once and declares the prototypes. Raises if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build the HIP library first "
                "(python -c 'import __graft_entry__ as g; g.build()')"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        vp, i32, sz = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t
        args_p = ctypes.POINTER(MoeFp8Args)
        lib.moe_fp8_workspace_bytes.argtypes = [i32]
        lib.moe_fp8_workspace_bytes.restype = sz
        lib.moe_fp8_workspace_layout.argtypes = [i32, ctypes.POINTER(MoeFp8Layout)]
        lib.moe_fp8_workspace_layout.restype = ctypes.c_int
        lib.moe_fp8_workspace_init.argtypes = [vp, sz, vp]
        lib.moe_fp8_workspace_init.restype = ctypes.c_int
        lib.moe_fp8_run.argtypes = [args_p, vp, sz, vp]
        lib.moe_fp8_run.restype = ctypes.c_int
        lib.moe_fp8_run_profiled.argtypes = [args_p, vp, sz, vp, sz, vp, ctypes.POINTER(vp)]
        lib.moe_fp8_run_profiled.restype = ctypes.c_int
        lib.moe_fp8_run_static.argtypes = [args_p, vp]
        lib.moe_fp8_run_static.restype = ctypes.c_int
        lib.moe_fp8_packed_weights_bytes.argtypes = []
        lib.moe_fp8_packed_weights_bytes.restype = sz
        lib.moe_fp8_pack_weights.argtypes = [args_p, vp, sz, vp]
        lib.moe_fp8_pack_weights.restype = ctypes.c_int
        lib.moe_fp8_run_packed.argtypes = [args_p, vp, sz, vp, sz, vp]
        lib.moe_fp8_run_packed.restype = ctypes.c_int
        lib.moe_fp8_route_dispatch.argtypes = [args_p, i32, vp, sz, vp]
        lib.moe_fp8_route_dispatch.restype = ctypes.c_int
        lib.moe_fp8_gemm1.argtypes = [args_p, vp, sz, vp]
        lib.moe_fp8_gemm1.restype = ctypes.c_int
        lib.moe_fp8_gemm2_combine.argtypes = [args_p, vp, sz, vp]
        lib.moe_fp8_gemm2_combine.restype = ctypes.c_int
        lib.moe_fp8_quantize_hidden.argtypes = [vp, i32, i32, vp, vp, vp]
        lib.moe_fp8_quantize_hidden.restype = ctypes.c_int
        lib.moe_fp8_strerror.argtypes = [ctypes.c_int]
        lib.moe_fp8_strerror.restype = ctypes.c_char_p
        lib.moe_fp8_version.argtypes = []
        lib.moe_fp8_version.restype = ctypes.c_char_p
        _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().moe_fp8_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code != OK:
        raise RuntimeError(f"{what} failed: {strerror(code)} (code {code})")


def workspace_layout(num_tokens: int) -> MoeFp8Layout:
    lay = MoeFp8Layout()
    check(load().moe_fp8_workspace_layout(int(num_tokens), ctypes.byref(lay)), "moe_fp8_workspace_layout")
    return lay


def workspace_bytes(num_tokens: int) -> int:
    return int(load().moe_fp8_workspace_bytes(int(num_tokens)))


def packed_weights_bytes() -> int:
    return int(load().moe_fp8_packed_weights_bytes())
