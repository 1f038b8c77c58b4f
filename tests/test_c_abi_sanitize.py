"""Host-side AddressSanitizer + UndefinedBehaviorSanitizer run of the C ABI.

The library's sources are compiled once more, into a temporary directory, with the two
sanitizers on the host side only (`-Xarch_host` before each `-fsanitize=`; the gfx950 device
code is built as for the product), and tests/c_abi_sanitize.c, a C caller built with clang and
the same sanitizers, walks every host path that runs without a GPU: workspace sizes and
layouts across the regime boundaries, every validation error of every entry point, the error
texts. Any sanitizer report aborts the program. Every call the program makes is rejected
before the library looks at the device, so it launches nothing. Leak checking is off: the
HIP runtime keeps allocations for the process's lifetime."""
import importlib.util
import os
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "mlsys26-flashinfer-moe_amd" / "csrc"
# the product build's per-file compiler flags (its build.py, loaded by path)
_spec = importlib.util.spec_from_file_location("_moe_fp8_build", CSRC.parent / "build.py")
_build = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(_build)
PER_FILE_FLAGS = _build.PER_FILE_FLAGS
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
CLANG = "/opt/rocm/llvm/bin/clang"
HOST_SAN = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
            "-Xarch_host", "-fno-omit-frame-pointer"]


@pytest.fixture(scope="module")
def sanitized_checker(tmp_path_factory):
    if not Path(HIPCC).exists() or not Path(CLANG).exists():
        pytest.skip("hipcc or the ROCm clang is not installed")
    d = tmp_path_factory.mktemp("asan")
    sources = sorted(CSRC.glob("*.hip"))

    def compile_one(src):
        extra = PER_FILE_FLAGS.get(src.name, [])
        cmd = [HIPCC, "--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", *HOST_SAN, *extra,
               "-c", str(src), "-o", str(d / (src.stem + ".o"))]
        return subprocess.run(cmd, capture_output=True, text=True)

    with ThreadPoolExecutor(max_workers=min(6, os.cpu_count() or 1)) as pool:
        for src, res in zip(sources, pool.map(compile_one, sources)):
            assert res.returncode == 0, f"{src.name}:\n{res.stdout}\n{res.stderr}"
    lib = d / "libmoe_fp8.so"
    res = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *HOST_SAN,
                          *map(str, sorted(d.glob("*.o"))), "-o", str(lib)], capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    exe = d / "c_abi_sanitize"
    res = subprocess.run([CLANG, "-std=c99", "-g", "-Wall", "-Wextra", "-Werror",
                          "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                          "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", f"-I{ROOT / 'include'}",
                          str(ROOT / "tests" / "c_abi_sanitize.c"), "-o", str(exe),
                          f"-L{d}", "-l:libmoe_fp8.so", f"-Wl,-rpath,{d}", "-Wl,-rpath,/opt/rocm/lib"],
                         capture_output=True, text=True)
    assert res.returncode == 0, res.stdout + res.stderr
    return exe


def test_c_abi_host_paths_are_sanitizer_clean(sanitized_checker):
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    res = subprocess.run([str(sanitized_checker)], capture_output=True, text=True, timeout=120, env=env)
    report = res.stdout + res.stderr
    assert "ERROR: AddressSanitizer" not in report and "runtime error:" not in report, report
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), report
