"""Seeded synthetic GGUF blocks and inputs for the benchmark configurations.

The reference builds its test and benchmark weights from seeded random bytes
(tests/make_tiny_model.py:87-172, tests/make_bench_model.py:112-118); these
generators do the same at the shapes of the benchmark configurations:

* Q8_0: int8 codes uniform in [-127, 127], d = fp16(|N(0, 0.02)|)
* Q4_K / Q5_K: d, dmin = fp16(|N(0, 1e-3)|); scale bytes, qh and qs uniform
  over 0..255 (which makes every 6-bit scale/min and every code uniform)
* Q6_K: ql / qh uniform, int8 scales uniform in [-32, 31], d = fp16(|N(0, 1e-3)|)
* Q4_0 / Q5_0: qs / qh uniform, d = fp16(|N(0, 1e-3)|); Q4_1 / Q5_1 add
  m = fp16(N(0, 1e-3))
* activations x ~ N(0, 1) in float32.
"""
from __future__ import annotations

import numpy as np

from .quants import QUANT_GEOMETRY


def _f16_bytes(vals: np.ndarray) -> np.ndarray:
    return vals.astype("<f2").view(np.uint8).reshape(-1, 2)


def random_blocks(dtype: str, rows: int, cols: int, seed: int = 0) -> np.ndarray:
    """(rows * cols / block_elements, block_bytes) uint8 of valid random blocks."""
    be, bb, _sub, _aff = QUANT_GEOMETRY[dtype]
    if cols % be:
        raise ValueError(f"{dtype}: cols must be a multiple of {be}")
    nb = rows * (cols // be)
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    if dtype == "Q8_0":
        b[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
        b[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb) * 0.02))
    elif dtype in ("Q4_K", "Q5_K"):
        b[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb) * 1e-3))
        b[:, 2:4] = _f16_bytes(np.abs(rng.standard_normal(nb) * 1e-3))
    elif dtype == "Q6_K":
        b[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = _f16_bytes(np.abs(rng.standard_normal(nb) * 1e-3))
    elif dtype in ("Q4_0", "Q5_0"):
        b[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb) * 1e-3))
    elif dtype in ("Q4_1", "Q5_1"):
        b[:, 0:2] = _f16_bytes(np.abs(rng.standard_normal(nb) * 1e-3))
        b[:, 2:4] = _f16_bytes(rng.standard_normal(nb) * 1e-3)
    else:
        raise ValueError(f"unsupported dtype {dtype}")
    return b


def random_matrix_bytes(dtype: str, rows: int, cols: int, seed: int = 0) -> bytes:
    return random_blocks(dtype, rows, cols, seed).tobytes()


def random_x(n: int, seed: int = 1, batch: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    shape = (n,) if batch is None else (batch, n)
    return rng.standard_normal(shape).astype(np.float32)
