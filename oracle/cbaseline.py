"""CPU baseline runners - TEST INFRASTRUCTURE (see oracle/__init__.py).

Two CPU legs for bench.py's cpu_baseline, both restatements of the
reference (the reference's own Python cannot be shipped to the GPU box):

* ``numpy_matvec``  - QuantMatrix.matvec's NumPy einsum path in the
  reference's order (alpacca/qmatrix.py:160-171), via qmatrix_ref.
* ``LoopMatvec``    - the C/OpenMP transliteration (matvec_loop.c) of the
  Numba-compiled fused loop (alpacca/kernels.py:49-69).
Both take the unpacked (codes, d_eff, m_eff) form that the reference builds
at load time; unpacking is outside the timed region, as in the reference.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BUILD = HERE / "_build"


def build() -> None:
    subprocess.run(["make", "-C", str(HERE), "-s"], check=True)


def _has_avx512() -> bool:
    try:
        flags = Path("/proc/cpuinfo").read_text()
    except OSError:
        return False
    return all(f in flags for f in ("avx512f", "avx512bw", "avx512dq", "avx512vl"))


def cores() -> int:
    return len(os.sched_getaffinity(0))


class LoopMatvec:
    """Numba-loop transliteration over the reference's unpacked layout."""

    def __init__(self, q3: np.ndarray, d: np.ndarray, m: np.ndarray | None):
        lib_path = BUILD / ("libmatvec_loop_v4.so" if _has_avx512() else "libmatvec_loop_v3.so")
        if not lib_path.exists():
            raise RuntimeError(f"{lib_path} not built (make -C oracle)")
        self.isa = lib_path.stem.rsplit("_", 1)[-1]
        self._lib = ctypes.CDLL(str(lib_path))
        fn = self._lib.matvec_codes
        fn.restype = None
        fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_int64,
                                              ctypes.c_void_p]
        self.q3 = np.ascontiguousarray(q3, dtype=np.int8)
        self.d = np.ascontiguousarray(d, dtype=np.float32)
        self.m = None if m is None else np.ascontiguousarray(m, dtype=np.float32)
        self.rows, self.nsub, self.sub = self.q3.shape

    def __call__(self, x: np.ndarray) -> np.ndarray:
        xs = np.ascontiguousarray(x, dtype=np.float32).reshape(self.nsub, self.sub)
        xsums = np.ascontiguousarray(xs.sum(axis=1), dtype=np.float32)
        out = np.empty(self.rows, dtype=np.float32)
        mp = self.m.ctypes.data if self.m is not None else self.d.ctypes.data
        self._lib.matvec_codes(self.q3.ctypes.data, self.d.ctypes.data, mp,
                               xs.ctypes.data, xsums.ctypes.data,
                               1 if self.m is not None else 0, self.rows,
                               self.nsub, self.sub, out.ctypes.data)
        return out
