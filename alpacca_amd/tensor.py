"""Dispatch seam: the reference's alpacca/tensor.py routing (tensor.py:28-47,
82-113) with QuantizedMatrix backed by the HIP library.  Dense NumPy weights
keep the reference's NumPy behaviour so that a model mixing dense and
quantized matrices routes exactly as before; dense weights uploaded with
dense_matrix() (F32/F16/BF16 in HBM) route to their methods like quantized
ones.
"""
from __future__ import annotations

import numpy as _np

from .qmatrix import (  # noqa: F401  (re-exported quantized-matrix surface)
    DENSE_DTYPES,
    QUANTIZED_MATVEC_DTYPES,
    DenseMatrix,
    QuantMatrix as QuantizedMatrix,
    _HBMMatrix,
    _reset_hot_cache_state,
    can_quantized_matvec,
    hot_cache_stats,
)
from .quants import QK, QK_K  # noqa: F401

HAS_NUMPY = True


def backend_name() -> str:
    return "hip-gfx950"


def quantized_matrix(data, dtype: str, rows: int, cols: int) -> QuantizedMatrix:
    return QuantizedMatrix(data, dtype, rows, cols)


def dense_matrix(data, dtype: str, rows: int, cols: int) -> DenseMatrix:
    """F32/F16/BF16 weights in HBM (the GGUF bytes, or an array of values)."""
    return DenseMatrix(data, dtype, rows, cols)


def is_quantized_matrix(W) -> bool:
    return isinstance(W, QuantizedMatrix)


def matvec(W, x):
    """W (rows x cols) times x (cols) -> rows."""
    if isinstance(W, _HBMMatrix):
        return W.matvec(x)
    return W @ x


def matmul_t(X, W):
    """X (batch x cols) times W.T (cols x rows) -> batch x rows."""
    if isinstance(W, _HBMMatrix):
        return W.matmul_t(X)
    return _np.asarray(X, dtype=_np.float32) @ W.T


def matrix_row(W, r: int):
    if isinstance(W, _HBMMatrix):
        return W.row(r)
    return W[r].copy()


def matrix_rows(W, rows):
    if isinstance(W, _HBMMatrix):
        return W.rows_at(rows)
    return W[_np.asarray(rows, dtype=_np.int64)].copy()
