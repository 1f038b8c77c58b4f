"""The C ABI from C: tests/c_abi_check.c, a C99 program, is compiled with gcc against
include/moe_fp8.h and linked with libmoe_fp8.so; the calls that need no GPU (struct sizes,
workspace sizes and layout, argument validation, error text) must agree with the ctypes
binding. This is the binding a C, cgo or other FFI caller makes."""
import ctypes
import shutil
import subprocess
from pathlib import Path

import pytest

import __graft_entry__ as ge

ROOT = Path(__file__).resolve().parent.parent


@pytest.fixture(scope="module")
def c_output(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc is not installed")
    ge.load_package()
    from mlsys26_flashinfer_moe_amd import _lib
    if not _lib.LIB_PATH.exists():
        pytest.skip("libmoe_fp8.so is not built")
    exe = tmp_path_factory.mktemp("c_abi") / "c_abi_check"
    libdir = _lib.LIB_PATH.parent
    cmd = ["gcc", "-std=c99", "-Wall", "-Wextra", "-Werror=implicit-function-declaration",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{ROOT / 'include'}",
           str(ROOT / "tests" / "c_abi_check.c"), "-o", str(exe),
           f"-L{libdir}", "-l:libmoe_fp8.so", f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=60).stdout
    return dict(line.split(" ", 1) for line in out.strip().splitlines())


def test_struct_sizes_match_ctypes(c_output):
    from mlsys26_flashinfer_moe_amd import _lib
    assert int(c_output["sizeof_args"]) == ctypes.sizeof(_lib.MoeFp8Args)
    assert int(c_output["sizeof_layout"]) == ctypes.sizeof(_lib.MoeFp8Layout)


def test_sizes_and_layout_match_ctypes(c_output):
    from mlsys26_flashinfer_moe_amd import _lib
    assert int(c_output["workspace_64"]) == _lib.workspace_bytes(64)
    assert int(c_output["workspace_8192"]) == _lib.workspace_bytes(8192)
    assert int(c_output["packed_bytes"]) == _lib.packed_weights_bytes()
    lay = _lib.workspace_layout(64)
    assert c_output["layout_rc"] == f"0 requant_block {lay.requant_block} rows_per_item {lay.rows_per_item}"


def test_argument_errors_through_c(c_output):
    from mlsys26_flashinfer_moe_amd import _lib
    rc, text = c_output["run_null"].split(" ", 1)
    assert int(rc) == _lib.EINVAL_POINTER and text == _lib.strerror(_lib.EINVAL_POINTER)
    assert int(c_output["run_negative"]) == _lib.EINVAL_TOKENS
    assert c_output["version"].startswith("moe_fp8 ")
