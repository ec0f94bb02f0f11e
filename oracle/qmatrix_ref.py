"""Oracle: QuantMatrix arithmetic (TEST INFRASTRUCTURE - see oracle/__init__.py).

* ``RefMatrix.matvec_ref``  - the reference's float32 matvec in its own order
  (alpacca/qmatrix.py:160-171: batched-matmul block dots below 2**20
  elements, einsum block dots otherwise, then the affine term
  m_eff @ sum(x_s)).
* ``RefMatrix.matmul_t_ref`` - the reference's tiled float32 prefill
  (qmatrix.py:196-211: ~4 MiB dequantized row tiles times X by BLAS, plus
  x_sub_sums @ m_eff.T).
* ``RefMatrix.matvec_f64`` / ``matmul_t_f64`` - float64 products over the
  exactly decoded weights: the tolerance anchor of the parity tests.
* ``RefMatrix.rows_at`` - decoded rows (qmatrix.py:232-246).
* ``quantize_x_q8`` / ``RefMatrix.matmul_t_int8_f64`` - the int8-activation
  prefill scheme of the Q8_0 MFMA path (no reference counterpart: the
  reference has no int8 activations): X per 32-element block, d = absmax/127
  (float32), q = rint(x / d) in float32; Y = sum_b d_x d_w (q_x . q_w) in
  float64.
* ``normalized_error`` - max_r |y_r - ref_r| / (||W_r|| * ||x||), the error
  measure of the north-star tolerances (2e-5 fp32, 1e-2 bf16 MFMA).
"""
from __future__ import annotations

import numpy as np

from .quants_ref import GEOMETRY, assemble, unpack

SMALL_MATVEC_ELEMS = 1 << 20  # qmatrix.py:55


class RefMatrix:
    def __init__(self, data, dtype: str, rows: int, cols: int):
        be, bb, sub, _aff = GEOMETRY[dtype]
        if cols % be:
            raise ValueError(f"{dtype} matrix columns must be a multiple of {be}")
        if len(data) != rows * (cols // be) * bb:
            raise ValueError("wrong byte length")
        self.dtype, self.rows, self.cols, self.sub = dtype, rows, cols, sub
        self.n_sub = cols // sub
        q, d, m = unpack(data, rows * cols, dtype)
        self.q3 = q.reshape(rows, self.n_sub, sub)
        self.d = d.reshape(rows, self.n_sub)
        self.m = None if m is None else m.reshape(rows, self.n_sub)
        self._q, self._d, self._m = q, d, m

    def dense(self) -> np.ndarray:
        """Decoded W, float32 (rows, cols) - bit-identical to quants.dequantize."""
        return assemble(self._q, self._d, self._m, self.sub).reshape(self.rows, self.cols)

    def rows_at(self, idx) -> np.ndarray:
        idx = np.asarray(idx, dtype=np.int64).reshape(-1)
        v = self.q3[idx].astype(np.float32)
        v *= self.d[idx][:, :, None]
        if self.m is not None:
            v += self.m[idx][:, :, None]
        return v.reshape(idx.size, self.cols)

    def matvec_ref(self, x) -> np.ndarray:
        xs = np.asarray(x, dtype=np.float32).reshape(self.n_sub, self.sub)
        if self.rows * self.cols < SMALL_MATVEC_ELEMS:
            q_small = np.ascontiguousarray(self.q3.transpose(1, 0, 2))
            blockdot = np.matmul(q_small.astype(np.float32), xs[:, :, None])[:, :, 0]
            out = np.einsum("sr,rs->r", blockdot, self.d)
        else:
            blockdot = np.einsum("rsl,sl->rs", self.q3, xs)
            out = np.einsum("rs,rs->r", blockdot, self.d)
        if self.m is not None:
            out += self.m @ xs.sum(axis=1)
        return out

    def matmul_t_ref(self, X) -> np.ndarray:
        X = np.asarray(X, dtype=np.float32)
        out = np.empty((X.shape[0], self.rows), dtype=np.float32)
        sums = None
        if self.m is not None:
            sums = X.reshape(X.shape[0], self.n_sub, self.sub).sum(axis=2)
        tile_rows = max(16, (4 << 20) // max(self.cols * 4, 1))
        for r0 in range(0, self.rows, tile_rows):
            r1 = min(self.rows, r0 + tile_rows)
            tile = np.ascontiguousarray(self.q3[r0:r1], dtype=np.float32)
            tile *= self.d[r0:r1, :, None]
            out[:, r0:r1] = X @ tile.reshape(r1 - r0, self.cols).T
            if self.m is not None:
                out[:, r0:r1] += sums @ self.m[r0:r1].T
        return out

    def matvec_f64(self, x) -> np.ndarray:
        return self.dense().astype(np.float64) @ np.asarray(x, dtype=np.float64)

    def matmul_t_f64(self, X) -> np.ndarray:
        return np.asarray(X, dtype=np.float64) @ self.dense().astype(np.float64).T

    def matmul_t_int8_f64(self, X) -> np.ndarray:
        """The int8 scheme (Q8_0 only): sum over blocks of d_x d_w times the
        exact integer block dot, in float64."""
        if self.dtype != "Q8_0":
            raise ValueError("the int8 scheme is defined for Q8_0 weights")
        qx, dx = quantize_x_q8(X)
        M = qx.shape[0]
        qx3 = qx.reshape(M, self.n_sub, 32).astype(np.int64)
        qw3 = self.q3.astype(np.int64)                       # (rows, n_sub, 32)
        dots = np.einsum("msk,rsk->mrs", qx3, qw3)          # exact integers
        return np.einsum("mrs,ms,rs->mr", dots.astype(np.float64), dx.astype(np.float64),
                         self.d.astype(np.float64))

    def row_norms(self) -> np.ndarray:
        return np.linalg.norm(self.dense().astype(np.float64), axis=1)


class DenseRef:
    """A dense F32/F16/BF16 matrix as the reference keeps it: decoded once to
    a float32 (rows, cols) array (model.py:276-281, quants.py:517-523) and
    multiplied by NumPy (tensor.py:82-97: W @ x, X @ W.T)."""

    def __init__(self, data, dtype: str, rows: int, cols: int):
        from .quants_ref import dense_decode
        self.dtype, self.rows, self.cols = dtype, rows, cols
        self.w = dense_decode(data, rows * cols, dtype).reshape(rows, cols)

    def dense(self) -> np.ndarray:
        return self.w

    def rows_at(self, idx) -> np.ndarray:
        return self.w[np.asarray(idx, dtype=np.int64).reshape(-1)].copy()

    def matvec_ref(self, x) -> np.ndarray:
        return self.w @ np.asarray(x, dtype=np.float32)

    def matmul_t_ref(self, X) -> np.ndarray:
        return np.asarray(X, dtype=np.float32) @ self.w.T

    def matvec_f64(self, x) -> np.ndarray:
        return self.w.astype(np.float64) @ np.asarray(x, dtype=np.float64)

    def matmul_t_f64(self, X) -> np.ndarray:
        return np.asarray(X, dtype=np.float64) @ self.w.astype(np.float64).T

    def row_norms(self) -> np.ndarray:
        return np.sqrt((self.w.astype(np.float64) ** 2).sum(axis=1))


def quantize_x_q8(X):
    """(q int8 (M, K), d float32 (M, K/32)): per 32-element block d =
    absmax / 127 and q = rint(x / d), both in float32; q = 0 where d = 0."""
    X = np.asarray(X, dtype=np.float32)
    M, K = X.shape
    b = X.reshape(M, K // 32, 32)
    d = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float32)
    safe = np.where(d > 0, d, np.float32(1.0))
    q = np.where(d[:, :, None] > 0, np.rint(b / safe[:, :, None]), 0).astype(np.int8)
    return q.reshape(M, K), d


def normalized_error(y, ref, row_norms, x) -> float:
    """max over outputs of |y - ref| / (||W_r|| * ||x||); x may be a batch
    (M, K), then each output (m, r) is normalized by ||W_r|| * ||X_m||."""
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    x = np.asarray(x, dtype=np.float64)
    if x.ndim == 1:
        den = row_norms * np.linalg.norm(x)
    else:
        den = np.linalg.norm(x, axis=1)[:, None] * row_norms[None, :]
    den = np.where(den > 0, den, 1.0)
    return float(np.max(np.abs(y - ref) / den)) if y.size else 0.0
