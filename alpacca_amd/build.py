"""Build libalpacca_amd.so (the HIP kernels + C ABI) in-tree for gfx950.

The shared library lands in ``alpacca_amd/_native/`` so that it travels with
the source tree; nothing is installed anywhere else.  ``python -m
alpacca_amd.build`` rebuilds it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
NATIVE = PKG / "_native"
LIB_NAME = "libalpacca_amd.so"
SOURCES = ("aq_api.hip", "aq_matvec.hip", "aq_matvec_i8.hip", "aq_dequant.hip",
           "aq_matmul.hip", "aq_matmul_h.hip", "aq_decode.hip", "aq_calibrate.hip")
ARCH = "gfx950"

# hipcc flags shared by every translation unit.  Packed fp32 VALU ops are
# disabled for the device pass (they are not used by hand and must not be
# formed by the compiler either).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
# Per-file additions.  The decode-step kernels and the one-segment decode
# matvec take their leading scalar arguments preloaded into scalar registers
# at wave launch (gfx950 kernel argument preloading): the kernels whose first
# memory operations depend on them skip the argument load's round trip.
FILE_FLAGS = {
    "aq_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "aq_matvec_i8.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("command failed: " + " ".join(cmd) + "\n" + r.stdout + r.stderr)


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    NATIVE.mkdir(exist_ok=True)
    obj_dir = NATIVE / "obj"
    obj_dir.mkdir(exist_ok=True)
    cc = hipcc()
    headers = sorted((PKG.parent / "include").glob("*.h")) + sorted(CSRC.glob("*.h"))

    def compile_one(src: str) -> Path:
        obj = obj_dir / (Path(src).stem + ".o")
        cmd = [cc, *HIPCC_FLAGS, *FILE_FLAGS.get(src, []), "-c", str(CSRC / src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), file=sys.stderr)
        _run(cmd)
        return obj

    with ThreadPoolExecutor(max_workers=min(6, len(SOURCES))) as ex:
        objs = list(ex.map(compile_one, SOURCES))
    del headers
    out = NATIVE / LIB_NAME
    tmp = NATIVE / (LIB_NAME + ".tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), file=sys.stderr)
    _run(cmd)
    os.replace(tmp, out)
    return out


def library_path() -> Path:
    return NATIVE / LIB_NAME


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
