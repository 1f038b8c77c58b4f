"""Builds libmoe_fp8.so (the C-ABI HIP library) in this package directory.

Every .hip source under csrc/ is compiled for gfx950 by hipcc into an object file
(in parallel) and the objects are linked into one shared library. Packed fp32 VALU
instructions are disabled for device code.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libmoe_fp8.so"
LIB_PATH = PKG_DIR / LIB_NAME
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# Routing must evaluate its fp32 operation sequence exactly as written.
PER_FILE_FLAGS = {
    "route_dispatch.hip": ["-ffp-contract=off"],
    # The tile GEMMs take their next work-list entry with a single-lane atomic whose result is
    # needed only at the end of the unit's epilogue; the atomic optimizer's rewrite reads the
    # result back at once, and that wait drains every load in flight.
    "gemm_tile.hip": ["-mllvm", "-amdgpu-atomic-optimizer-strategy=None"],
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build libmoe_fp8")
    return exe


def build(verbose: bool = False) -> Path:
    """Compiles every csrc/*.hip for gfx950 and links LIB_PATH. Always rebuilds."""
    OBJ_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    cc = hipcc()
    procs = []
    objs = []
    for src in sources:
        obj = OBJ_DIR / (src.stem + ".o")
        objs.append(obj)
        cmd = [cc, *COMMON_FLAGS, *PER_FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, proc in procs:
        out, _ = proc.communicate()
        text = out.decode(errors="replace")
        # hipcc's host pass does not know the device-only feature flag; that note is harmless.
        text = "\n".join(l for l in text.splitlines() if "packed-fp32-ops" not in l)
        if proc.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text, flush=True)
    if failed:
        msg = "\n".join(f"--- {s.name} ---\n{t}" for s, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError("link failed:\n" + res.stdout.decode(errors="replace"))
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
