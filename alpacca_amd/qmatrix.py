"""QuantMatrix: GGUF-quantized weights resident in HBM, drop-in for the
reference's alpacca.qmatrix.QuantMatrix (alpacca/qmatrix.py:64).

Same constructor, attributes, methods and exceptions as the reference:

* ``QuantMatrix(data, dtype, rows, cols)`` copies the raw GGUF blocks to the
  GPU once; the caller's buffer (often a memoryview into an mmap that closes
  right after loading, model.py:340-341) is not retained.  ValueError for an
  unsupported dtype, a column count that is not a multiple of the block, or a
  wrong byte length (qmatrix.py:78-96).
* ``matvec(x)`` / ``W @ x`` -> float32 (rows,)            (qmatrix.py:145-171)
* ``matmul_t(X)`` -> X @ W.T, float32 (batch, rows)      (qmatrix.py:184-211)
* ``row(i)`` / ``rows_at(idx)`` -> decoded float32 rows, IndexError when out
  of range (qmatrix.py:215-246)
* ``shape``, ``storage_nbytes()``, ``dtype``, ``rows``, ``cols``,
  ``block_elements``, ``block_bytes``, ``blocks_per_row``, ``sub_len``,
  ``n_sub``, ``data`` (None: nothing is kept on the host).

Host NumPy arrays in and out keep the reference's calling convention (the
call copies x to HBM, runs the kernel, copies y back and waits).  Device
tensors (a torch tensor on the GPU, or raw device pointers through
``matvec_device``/``matmul_t_device``) stay on the device and only enqueue.

Differences from the reference, by design: there is no host-side dense "hot
cache" (ALPACCA_HOT_WEIGHT_MB, qmatrix.py:248-347) - the weights are already
in HBM, so hot_cache_stats() always reports zero usage.  matmul_t keeps
the reference's float32 products by default (within the reference's own
batched-vs-sequential bar, tests/smoke.py:950-972); precision="bf16" (or
ALPACCA_PREFILL_PRECISION=bf16) opts into bf16 matrix cores (1e-2 bar), and
precision="int8" into int8 activations for Q8_0.
"""
from __future__ import annotations

import ctypes
import os
import weakref

import numpy as np

from . import _lib
from .quants import QUANT_GEOMETRY

QUANTIZED_MATVEC_DTYPES = frozenset(QUANT_GEOMETRY)


def _destroy(handle: int) -> None:
    try:
        _lib.load().aq_matrix_destroy(ctypes.c_void_p(handle))
    except Exception:  # pragma: no cover - interpreter shutdown
        pass


def _is_device_tensor(v) -> bool:
    return getattr(v, "is_cuda", False) is True


def _torch_stream(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream


def _layout_id(layout) -> int:
    name = (layout or os.environ.get("ALPACCA_AMD_LAYOUT", "auto")).lower()
    if name not in _lib.LAYOUT_IDS:
        raise ValueError(f"unknown layout {name!r} (auto, raw, split)")
    return _lib.LAYOUT_IDS[name]


def _matvec_flags(kernel) -> int:
    if kernel is None and "ALPACCA_AMD_MATVEC" not in os.environ:
        return 0  # the default int8 kernel
    name = (kernel or os.environ.get("ALPACCA_AMD_MATVEC", "int8")).lower()
    if name not in ("int8", "fp32"):
        raise ValueError(f"unknown matvec kernel {name!r} (int8, fp32)")
    return _lib.AQ_MATVEC_FP32 if name == "fp32" else 0


def _prec_id(precision) -> int:
    name = (precision or os.environ.get("ALPACCA_PREFILL_PRECISION", "auto")).lower()
    if name not in _lib.PREC_IDS:
        raise ValueError(f"unknown precision {name!r} (auto, fp32, bf16, int8)")
    return _lib.PREC_IDS[name]


class _HBMMatrix:
    """A (rows x cols) weight matrix resident in HBM behind the C ABI; the
    methods shared by QuantMatrix and DenseMatrix."""

    __slots__ = ("dtype", "rows", "cols", "block_elements", "block_bytes",
                 "blocks_per_row", "sub_len", "n_sub", "data", "layout",
                 "_handle", "_finalizer", "__weakref__")

    def _create(self, data, dtype: str, rows: int, cols: int, layout,
                block_elements: int, block_bytes: int, sub_len: int) -> None:
        self.dtype = dtype
        self.rows = rows
        self.cols = cols
        self.block_elements = block_elements
        self.block_bytes = block_bytes
        self.blocks_per_row = cols // block_elements
        self.sub_len = sub_len
        self.n_sub = cols // sub_len
        self._handle = None
        self._finalizer = None
        expected = rows * self.blocks_per_row * block_bytes
        if len(data) != expected:
            raise ValueError(
                f"{dtype} matrix has {len(data)} bytes, expected {expected}")
        lib = _lib.ensure_device()
        buf = np.frombuffer(data, dtype=np.uint8) if expected else np.zeros(1, np.uint8)
        handle = ctypes.c_void_p()
        _lib.check(lib.aq_matrix_create(
            ctypes.c_void_p(buf.ctypes.data), expected, _lib.DTYPE_IDS[dtype],
            rows, cols, _layout_id(layout), ctypes.byref(handle)))
        self._handle = handle.value
        self._finalizer = weakref.finalize(self, _destroy, handle.value)
        lay = ctypes.c_int(0)
        _lib.check(lib.aq_matrix_info(ctypes.c_void_p(self._handle), None, None,
                                      None, ctypes.byref(lay), None))
        self.layout = {1: "raw", 2: "split"}[lay.value]
        self.data = None  # the HBM copy owns everything

    # ---- introspection ---------------------------------------------------

    def __repr__(self) -> str:
        return f"{type(self).__name__}({self.dtype}, {self.rows}x{self.cols})"

    @property
    def shape(self) -> tuple[int, int]:
        return self.rows, self.cols

    def storage_nbytes(self) -> int:
        """Bytes of HBM holding the quantized matrix: its one allocation, the
        GGUF blocks (raw layout) or the split planes each padded to 256 bytes."""
        n = ctypes.c_size_t(0)
        _lib.check(_lib.load().aq_matrix_info(ctypes.c_void_p(self._handle), None,
                                              None, None, None, ctypes.byref(n)))
        return n.value

    @property
    def handle(self) -> int:
        """The aq_matrix* of the C ABI (for device-resident callers)."""
        return self._handle

    # ---- matvec (decode path) ---------------------------------------------

    def __matmul__(self, x):
        return self.matvec(x)

    def matvec(self, x, kernel=None):
        """self (rows x cols) @ x (cols) -> (rows).

        kernel: "int8" (default; x split into three int8 pieces per 32-group,
        exact integer dot products) or "fp32" (fp32 FMA on exact fp32 x);
        ALPACCA_AMD_MATVEC sets the default."""
        lib = _lib.load()
        if _is_device_tensor(x):
            import torch
            if x.numel() != self.cols:
                raise ValueError(f"expected {self.cols} inputs, got {x.numel()}")
            xd = x.reshape(-1).to(torch.float32).contiguous()
            y = torch.empty(self.rows, dtype=torch.float32, device=xd.device)
            self.matvec_device(xd.data_ptr(), y.data_ptr(), _torch_stream(xd), kernel)
            return y
        # a float32 vector already in the layout the call needs goes as it is
        # (the per-call Python work is part of every host-array call)
        if (type(x) is np.ndarray and x.dtype == np.float32 and x.ndim == 1
                and x.flags.c_contiguous):
            xs = x
        else:
            xs = np.ascontiguousarray(np.asarray(x, dtype=np.float32).reshape(-1))
        if xs.size != self.cols:
            raise ValueError(f"expected {self.cols} inputs, got {xs.size}")
        y = np.empty(self.rows, dtype=np.float32)
        rc = lib.aq_matvec(self._handle, xs.__array_interface__["data"][0],
                           y.__array_interface__["data"][0],
                           _matvec_flags(kernel), None)
        if rc:
            _lib.check(rc)
        return y

    def matvec_device(self, x_ptr: int, y_ptr: int, stream: int = 0,
                      kernel=None) -> None:
        """Enqueue y = W x on `stream` for device pointers x (cols) / y (rows)."""
        _lib.check(_lib.load().aq_matvec(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(x_ptr),
            ctypes.c_void_p(y_ptr),
            _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE | _matvec_flags(kernel),
            ctypes.c_void_p(stream)))

    # ---- batched matmul (prefill path) -------------------------------------

    def matmul_t(self, X, precision=None):
        """X (batch x cols) @ self.T -> (batch x rows)."""
        if _is_device_tensor(X):
            import torch
            if X.dim() != 2 or X.shape[1] != self.cols:
                raise ValueError(
                    f"expected (batch, {self.cols}) input, got {tuple(X.shape)}")
            Xd = X.to(torch.float32).contiguous()
            Y = torch.empty((Xd.shape[0], self.rows), dtype=torch.float32,
                            device=Xd.device)
            self.matmul_t_device(Xd.data_ptr(), Xd.shape[0], Y.data_ptr(),
                                 _torch_stream(Xd), precision)
            return Y
        X = np.asarray(X, dtype=np.float32)
        if X.ndim != 2 or X.shape[1] != self.cols:
            lead = X.shape[0] if X.ndim else 0
            raise ValueError(
                f"expected ({lead}, {self.cols}) input, got {X.shape}")
        X = np.ascontiguousarray(X)
        Y = np.empty((X.shape[0], self.rows), dtype=np.float32)
        _lib.check(_lib.load().aq_matmul_t(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(X.ctypes.data),
            X.shape[0], ctypes.c_void_p(Y.ctypes.data), _prec_id(precision), 0,
            None))
        return Y

    def matmul_t_device(self, X_ptr: int, M: int, Y_ptr: int, stream: int = 0,
                        precision=None) -> None:
        """Enqueue Y = X W^T on `stream` for device pointers X (M x cols)."""
        _lib.check(_lib.load().aq_matmul_t(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(X_ptr), int(M),
            ctypes.c_void_p(Y_ptr), _prec_id(precision),
            _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE, ctypes.c_void_p(stream)))

    def matmul_t_swiglu_device(self, X_ptr: int, M: int, Z_ptr: int, out_ptr: int,
                               stream: int = 0, precision=None) -> None:
        """Enqueue out = silu(Z[:, 0::2]) * Z[:, 1::2] for Z = X W^T, rows of W
        being interleaved (gate, up) pairs (model.py:511-513); Z (M x rows)
        is scratch that the library may leave unwritten."""
        _lib.check(_lib.load().aq_matmul_t_swiglu(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(X_ptr), int(M),
            ctypes.c_void_p(Z_ptr), ctypes.c_void_p(out_ptr), _prec_id(precision),
            _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE, ctypes.c_void_p(stream)))

    # ---- row access (embedding lookups) ------------------------------------

    def row(self, i: int):
        if not 0 <= i < self.rows:
            raise IndexError(i)
        return self.rows_at([i])[0]

    def rows_at(self, rows):
        idx = np.ascontiguousarray(np.asarray(rows, dtype=np.int64).reshape(-1))
        if idx.size and (int(idx.min()) < 0 or int(idx.max()) >= self.rows):
            raise IndexError("row index out of range")
        out = np.empty((idx.size, self.cols), dtype=np.float32)
        _lib.check(_lib.load().aq_dequant_rows(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(idx.ctypes.data),
            idx.size, ctypes.c_void_p(out.ctypes.data), 0, None))
        return out

    def rows_at_device(self, idx_ptr: int, n: int, out_ptr: int,
                       stream: int = 0) -> None:
        """Enqueue the gather of n device-resident int64 row indices (clamped
        to [0, rows) - a kernel cannot raise IndexError) into out (n x cols)."""
        _lib.check(_lib.load().aq_dequant_rows(
            ctypes.c_void_p(self._handle), ctypes.c_void_p(idx_ptr), int(n),
            ctypes.c_void_p(out_ptr), _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE,
            ctypes.c_void_p(stream)))


class QuantMatrix(_HBMMatrix):
    """Quantized (rows x cols) matrix in HBM; quant blocks run along columns."""

    __slots__ = ()

    def __init__(self, data, dtype: str, rows: int, cols: int, layout=None):
        geom = QUANT_GEOMETRY.get(dtype)
        if geom is None:
            raise ValueError(f"quantized matvec does not support {dtype}")
        block_elements, block_bytes, sub_len, _affine = geom
        if cols % block_elements:
            raise ValueError(
                f"{dtype} matrix columns must be a multiple of {block_elements}")
        self._create(data, dtype, rows, cols, layout, block_elements, block_bytes, sub_len)


# dense values per dtype: bytes per value
DENSE_DTYPES = {"F32": 4, "F16": 2, "BF16": 2}
DENSE_BLOCK = 32  # values per block along K in the library's dense layout


class DenseMatrix(_HBMMatrix):
    """F32 / F16 / BF16 weights kept in HBM as stored - the reference's dense
    fallback (model.py:269-281 dequantizes them to a float32 ndarray and
    multiplies with NumPy).  Same methods as QuantMatrix; matvec always runs
    the fp32 kernel, matmul_t the MFMA path (fp32 products unless bf16 is
    asked for, as for QuantMatrix), row gathers decode exactly
    (quants.py:517-523).
    ValueError for another dtype, a column count that is not a multiple of
    32 (the library's block along K) or a wrong byte length."""

    __slots__ = ()

    def __init__(self, data, dtype: str, rows: int, cols: int):
        width = DENSE_DTYPES.get(dtype)
        if width is None:
            raise ValueError(f"dense matrices are F32, F16 or BF16, not {dtype}")
        if cols % DENSE_BLOCK:
            raise ValueError(f"{dtype} matrix columns must be a multiple of {DENSE_BLOCK}")
        if isinstance(data, np.ndarray):  # values (or their bytes) as an array
            data = np.ascontiguousarray(data).reshape(-1).view(np.uint8)
        self._create(data, dtype, rows, cols, None, DENSE_BLOCK, DENSE_BLOCK * width,
                     DENSE_BLOCK)


# dtype pairs one multi launch may mix (matrices of the first dtype first);
# the same list as aq::matvec_mixed_supported in the C ABI
MIXABLE_DTYPES = frozenset({("Q4_K", "Q6_K"), ("Q5_K", "Q6_K"), ("Q4_K", "Q5_K")})


def matvec_multi_device(mats, x_ptr: int, y_ptrs, stream: int = 0) -> None:
    """Enqueue y_i = W_i x for up to 8 QuantMatrix objects sharing x (same
    dtype, cols and layout) as ONE kernel launch - the fused form of the
    reference's per-projection matvecs on one input (model.py:529-531 q/k/v,
    :549-550 gate/up).  x and y_i are device pointers."""
    mats = list(mats)
    ys = list(y_ptrs)
    if not 1 <= len(mats) <= 8 or len(ys) != len(mats):
        raise ValueError("matvec_multi_device takes 1..8 matrices and as many outputs")
    hs = (ctypes.c_void_p * len(mats))(*[m._handle for m in mats])
    yp = (ctypes.c_void_p * len(ys))(*ys)
    _lib.check(_lib.load().aq_matvec_multi(
        hs, len(mats), ctypes.c_void_p(x_ptr), yp,
        _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE, ctypes.c_void_p(stream)))


def matvec_fused_device(mats, x_ptr: int, y_ptrs, stream: int = 0, *, x2_ptr: int = 0,
                        norm_w_ptr: int = 0, eps: float = 0.0, rmsnorm: bool = False,
                        swiglu: bool = False, accumulate: bool = False,
                        swiglu_pairs: bool = False) -> None:
    """matvec_multi_device with the decode step's elementwise work folded in
    (aq_matvec_fused): rmsnorm=True uses x * inv * norm_w as the input,
    swiglu=True uses x / (1 + exp(-x)) * x2, accumulate=True adds W x to the
    outputs instead of overwriting them, swiglu_pairs=True treats the rows
    as (gate, up) pairs (interleave_rows) and writes silu(gate) * up, one
    output per pair.  Outputs must not overlap x or x2."""
    mats = list(mats)
    ys = list(y_ptrs)
    if not 1 <= len(mats) <= 8 or len(ys) != len(mats):
        raise ValueError("matvec_fused_device takes 1..8 matrices and as many outputs")
    flags = _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE
    flags |= (_lib.AQ_X_RMSNORM if rmsnorm else 0) | (_lib.AQ_X_SWIGLU if swiglu else 0)
    flags |= _lib.AQ_Y_ACCUMULATE if accumulate else 0
    flags |= _lib.AQ_Y_SWIGLU_PAIRS if swiglu_pairs else 0
    hs = (ctypes.c_void_p * len(mats))(*[m._handle for m in mats])
    yp = (ctypes.c_void_p * len(ys))(*ys)
    _lib.check(_lib.load().aq_matvec_fused(
        hs, len(mats), ctypes.c_void_p(x_ptr), ctypes.c_void_p(x2_ptr),
        ctypes.c_void_p(norm_w_ptr), ctypes.c_float(eps), yp, flags,
        ctypes.c_void_p(stream)))


def pair_rows_supported(dtype: str, cols: int) -> bool:
    """Rows of this dtype and width run two per wave in the integer kernel
    (at most 32 lane units: 64 values per unit for the K-quants, 32 for the
    32-element formats) - what swiglu_pairs needs."""
    geom = QUANT_GEOMETRY.get(dtype)
    if geom is None or cols % geom[0]:
        return False
    return cols // (64 if geom[0] == 256 else 32) <= 32


def interleave_rows(a, b, rows: int, cols: int, dtype: str) -> np.ndarray:
    """The GGUF bytes of two (rows x cols) matrices of one dtype as one
    (2 rows x cols) matrix with rows a0, b0, a1, b1, ... (uint8 array)."""
    be, bb = QUANT_GEOMETRY[dtype][:2]
    rb = cols // be * bb
    A = np.frombuffer(a, dtype=np.uint8).reshape(rows, rb)
    B = np.frombuffer(b, dtype=np.uint8).reshape(rows, rb)
    return np.stack([A, B], axis=1).reshape(-1)


def hot_cache_stats() -> dict[str, int]:
    """The reference's host dense-cache counters (qmatrix.py:340-347); the
    weights live in HBM here, so no host cache is ever built."""
    return {"limit_bytes": 0, "used_bytes": 0, "matrices": 0}


def _reset_hot_cache_state() -> None:
    """No host cache to reset (reference: qmatrix.py:334-337)."""


def can_quantized_matvec(dtype: str, cols: int) -> bool:
    geom = QUANT_GEOMETRY.get(dtype)
    return geom is not None and cols % geom[0] == 0


QMatrix = QuantMatrix

__all__ = ["QuantMatrix", "QMatrix", "DenseMatrix", "DENSE_DTYPES",
           "QUANTIZED_MATVEC_DTYPES", "can_quantized_matvec", "hot_cache_stats"]
