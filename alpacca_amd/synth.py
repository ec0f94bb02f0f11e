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


# ---------------------------------------------------------------------------
# Synthetic model weights (config 5).  The block recipes above give every
# Q4_K weight a large positive mean (codes 0..15 times d*sc, minus a min of
# the same order), which would make all logits of a random model move
# together and greedy decoding repeat one token.  Model weights are instead
# drawn with zero mean and a chosen standard deviation, like the reference's
# bench models (tests/make_bench_model.py:112-118 draws N(0, 0.02) and
# quantizes); the blocks are generated directly in quantized form:
#
# * Q4_K: codes uniform 0..15, 6-bit scales sc uniform in 32..63, mins
#   mn = round(15 sc / 16), dmin = 8 d exactly, so w = d sc q - 8 d mn
#   ~= d sc (q - 7.5): zero mean, std ~= 224 d;
# * Q6_K: codes uniform (q - 32 in -32..31), int8 scales uniform in -32..31,
#   std ~= 342 d;
# * per block d = std / (224 or 342) * U(0.5, 1.5), stored as fp16.

def pack_kquant_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """(nb, 8) six-bit scales and mins -> (nb, 12) packed bytes, the inverse
    of the Q4_K/Q5_K scale unpacking (alpacca/quants.py:127-133)."""
    sc = np.asarray(sc, dtype=np.uint8)
    mn = np.asarray(mn, dtype=np.uint8)
    out = np.empty((sc.shape[0], 12), dtype=np.uint8)
    out[:, 0:4] = sc[:, 0:4] | ((sc[:, 4:8] >> 4) << 6)
    out[:, 4:8] = mn[:, 0:4] | ((mn[:, 4:8] >> 4) << 6)
    out[:, 8:12] = (sc[:, 4:8] & 15) | ((mn[:, 4:8] & 15) << 4)
    return out


def model_blocks(dtype: str, rows: int, cols: int, seed: int, std: float = 0.02) -> np.ndarray:
    """Zero-mean weight blocks of standard deviation ~std (Q4_K or Q6_K)."""
    be, bb, _sub, _aff = QUANT_GEOMETRY[dtype]
    if cols % be:
        raise ValueError(f"{dtype}: cols must be a multiple of {be}")
    nb = rows * (cols // be)
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    spread = rng.uniform(0.5, 1.5, nb)
    if dtype == "Q4_K":
        d = (std / 224.0 * spread).astype(np.float16)
        sc = rng.integers(32, 64, size=(nb, 8), dtype=np.uint8)
        mn = ((sc.astype(np.uint16) * 15 + 8) // 16).astype(np.uint8)
        b[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        b[:, 2:4] = (d.astype(np.float32) * 8).astype(np.float16).view(np.uint8).reshape(-1, 2)
        b[:, 4:16] = pack_kquant_scales(sc, mn)
    elif dtype == "Q6_K":
        b[:, 192:208] = rng.integers(-32, 32, size=(nb, 16), dtype=np.int8).view(np.uint8)
        b[:, 208:210] = (std / 342.0 * spread).astype(np.float16).view(np.uint8).reshape(-1, 2)
    else:
        raise ValueError(f"model_blocks supports Q4_K and Q6_K, not {dtype}")
    return b


def dense_values_bytes(dtype: str, rows: int, cols: int, seed: int = 0,
                       std: float = 0.02) -> np.ndarray:
    """Dense weights N(0, std) stored as F32, F16 or BF16 (round to nearest
    even), as the little-endian bytes a GGUF file holds (uint8 array)."""
    v = np.random.default_rng(seed).standard_normal(rows * cols).astype(np.float32) * np.float32(std)
    if dtype == "F32":
        return v.astype("<f4").view(np.uint8)
    if dtype == "F16":
        return v.astype("<f2").view(np.uint8)
    if dtype == "BF16":
        b = v.view(np.uint32).astype(np.uint64)
        r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype("<u2")
        return r.view(np.uint8)
    raise ValueError(f"not a dense dtype: {dtype}")
