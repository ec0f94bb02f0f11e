"""matmul_t on the exact-integer fp16 kernel (aq_matmul_h.hip: Q4_K weights as
sc*code integers, Q6_K weights as q - 32 with d*sc per 16-element group in
fp32, on fp16 matrix cores, X in two fp16 pieces after a per-row
power-of-two scale, d and dmin applied in fp32) against the float64 oracle
(oracle/qmatrix_ref.py, the reference's QuantMatrix.matmul_t,
alpacca/qmatrix.py:184-211).  Bar: 2e-5 normalized by ||W_r|| * ||x_m||, the
north star's fp32 tolerance."""
from __future__ import annotations

import numpy as np
import pytest

from alpacca_amd import synth
from alpacca_amd.qmatrix import QuantMatrix
from oracle import quants_ref as Q
from oracle.qmatrix_ref import RefMatrix, normalized_error

pytestmark = pytest.mark.gpu

FP32_TOL = 2e-5


def _f64(data, rows, cols, X, dtype="Q4_K"):
    W = Q.dequantize(data, rows * cols, dtype).reshape(rows, cols).astype(np.float64)
    return np.asarray(X, dtype=np.float64) @ W.T, np.linalg.norm(W, axis=1)


def _adversarial_q4k(rows, cols, seed):
    """Random bytes everywhere; d and dmin finite fp16 of either sign, normal
    and subnormal (the kernel's B operand is sc*code whatever the header)."""
    nb = rows * cols // 256
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, 144), dtype=np.uint8)
    for o in (0, 2):
        mag = 10.0 ** rng.uniform(-7.5, 0.5, nb)
        sign = rng.choice([-1.0, 1.0], nb)
        b[:, o:o + 2] = (mag * sign).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b.tobytes()


@pytest.mark.parametrize("layout", ["raw", "split"])
@pytest.mark.parametrize("precision", ["auto", "fp32"])
@pytest.mark.parametrize("M,rows,cols", [(3, 1000, 4096), (5, 300, 2048), (8, 512, 2048),
                                         (16, 4096, 4096), (37, 1000, 2048),
                                         (64, 300, 4096), (130, 700, 4096), (513, 256, 2048),
                                         (128, 4096, 14336)])
def test_exact_fp16_matmul_vs_f64(M, rows, cols, precision, layout):
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=rows + M)
    X = synth.random_x(cols, seed=M, batch=M)
    qm = QuantMatrix(data, "Q4_K", rows, cols, layout=layout)
    want, norms = _f64(data, rows, cols, X)
    err = normalized_error(qm.matmul_t(X, precision=precision), want, norms, X)
    assert err < FP32_TOL, err


@pytest.mark.parametrize("M", [8, 100])
def test_exact_fp16_adversarial_blocks(M):
    rows, cols = 384, 2048
    data = _adversarial_q4k(rows, cols, seed=M)
    X = synth.random_x(cols, seed=M + 1, batch=M)
    want, norms = _f64(data, rows, cols, X)
    for prec in ("auto", "fp32"):
        err = normalized_error(QuantMatrix(data, "Q4_K", rows, cols).matmul_t(X, precision=prec),
                               want, norms, X)
        assert err < FP32_TOL, (prec, err)


def test_exact_fp16_x_magnitudes():
    """Rows of zeros, of 1e30, of 1e-30 and of mixed magnitudes (1e-20 beside
    1e20): the per-row scale keeps every row in range."""
    rows, cols, M = 512, 2048, 72
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=3)
    X = synth.random_x(cols, seed=4, batch=M)
    X[0] = 0
    X[1] *= 1e30
    X[2] *= 1e-30
    X[3, ::2] *= 1e-20
    X[3, 1::2] *= 1e20
    X[4, :32] = 1e25  # one sub-block far above the rest
    want, norms = _f64(data, rows, cols, X)
    for prec in ("auto", "fp32"):
        Y = QuantMatrix(data, "Q4_K", rows, cols).matmul_t(X, precision=prec)
        assert np.all(Y[0] == 0)
        err = normalized_error(Y, want, norms, X)
        assert err < FP32_TOL, (prec, err)


def test_exact_fp16_bits_do_not_depend_on_m():
    """precision fp32 (the batched prefill step's): every output is the same
    sequence of operations for any M, so slices of X give the rows of the
    whole product bit for bit."""
    rows, cols = 700, 4096
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=9)
    qm = QuantMatrix(data, "Q4_K", rows, cols)
    X = synth.random_x(cols, seed=10, batch=150)
    whole = qm.matmul_t(X, precision="fp32")
    parts = np.concatenate([qm.matmul_t(X[a:b], precision="fp32")
                            for a, b in ((0, 7), (7, 71), (71, 150))])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))


def test_exact_fp16_nonfinite_rows():
    """A NaN or an infinity in a row of X makes that row's outputs non-finite
    and leaves the other rows correct."""
    rows, cols, M = 256, 2048, 16
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=5)
    X = synth.random_x(cols, seed=6, batch=M)
    X[3, 100] = np.nan
    X[7, 5] = np.inf
    Y = QuantMatrix(data, "Q4_K", rows, cols).matmul_t(X, precision="auto")
    assert not np.isfinite(Y[3]).any() and not np.isfinite(Y[7]).any()
    keep = [i for i in range(M) if i not in (3, 7)]
    want, norms = _f64(data, rows, cols, X[keep])
    assert normalized_error(Y[keep], want, norms, X[keep]) < FP32_TOL


def test_exact_fp16_matches_reference_order():
    """The reference's own float32 matmul_t order (qmatrix.py:196-211: f32 row
    tiles of d*q, BLAS, plus the min term) agrees to the same bar."""
    rows, cols, M = 600, 2048, 96
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=12)
    X = synth.random_x(cols, seed=13, batch=M)
    ref = RefMatrix(data, "Q4_K", rows, cols)
    Y = QuantMatrix(data, "Q4_K", rows, cols).matmul_t(X)
    assert normalized_error(Y, ref.matmul_t_ref(X).astype(np.float64), ref.row_norms(), X) < FP32_TOL


def _with_env(name, fn):
    import os
    os.environ[name] = "1"
    try:
        return fn()
    finally:
        del os.environ[name]


@pytest.mark.parametrize("M,rows,cols", [(8, 1000, 4096), (16, 4096, 4096), (13, 300, 14336)])
def test_exact_fp16_fused_x_matches_prepared_x(M, rows, cols):
    """Up to 16 rows the workgroups cut X into fp16 pieces themselves, with a
    power-of-two scale per row over their split's columns.  For X of
    ordinary range that is the prepared pieces shifted by a power of two, so
    the outputs equal those of the two-launch form (AQ_MATMUL_X_PREP) bit for
    bit."""
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=rows + M)
    qm = QuantMatrix(data, "Q4_K", rows, cols)
    X = synth.random_x(cols, seed=M, batch=M)
    prepared = _with_env("AQ_MATMUL_X_PREP", lambda: qm.matmul_t(X))
    assert np.array_equal(qm.matmul_t(X).view(np.uint32), prepared.view(np.uint32))


def test_exact_fp16_fused_x_magnitudes():
    """The fused staging at 16 rows with rows of zeros, of 1e30, of 1e-30, of
    1e-20 beside 1e20 and with one sub-block far above the rest (per-split
    scales: each split's maximum sets its own)."""
    rows, cols, M = 1024, 4096, 16
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=31)
    X = synth.random_x(cols, seed=32, batch=M)
    X[0] = 0
    X[1] *= 1e30
    X[2] *= 1e-30
    X[3, ::2] *= 1e-20
    X[3, 1::2] *= 1e20
    X[4, :32] = 1e25
    X[5, 2048:] = 0  # a split of zeros beside splits of values
    want, norms = _f64(data, rows, cols, X)
    Y = QuantMatrix(data, "Q4_K", rows, cols).matmul_t(X)
    assert np.all(Y[0] == 0)
    assert normalized_error(Y, want, norms, X) < FP32_TOL


# ---- Q6_K: q - 32 on the matrix cores, d * sc per 16-element group in fp32 ----

def _adversarial_q6k(rows, cols, seed):
    """Random bytes everywhere (codes, and int8 scales over the whole range
    -128..127); d a finite fp16 of either sign, normal and subnormal."""
    nb = rows * cols // 256
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, 210), dtype=np.uint8)
    mag = 10.0 ** rng.uniform(-7.5, 0.5, nb)
    b[:, 208:210] = (mag * rng.choice([-1.0, 1.0], nb)).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b.tobytes()


@pytest.mark.parametrize("precision", ["auto", "fp32"])
@pytest.mark.parametrize("M,rows,cols", [(64, 300, 2048), (130, 1000, 4096), (513, 256, 2048),
                                         (128, 2048, 8192), (70, 4096, 14336)])
def test_exact_fp16_q6k_vs_f64(M, rows, cols, precision):
    data = synth.random_matrix_bytes("Q6_K", rows, cols, seed=rows + M)
    X = synth.random_x(cols, seed=M, batch=M)
    want, norms = _f64(data, rows, cols, X, "Q6_K")
    err = normalized_error(QuantMatrix(data, "Q6_K", rows, cols).matmul_t(X, precision=precision),
                           want, norms, X)
    assert err < FP32_TOL, err


@pytest.mark.parametrize("M", [8, 100])
def test_exact_fp16_q6k_adversarial_blocks(M):
    rows, cols = 384, 2048
    data = _adversarial_q6k(rows, cols, seed=M)
    X = synth.random_x(cols, seed=M + 1, batch=M)
    want, norms = _f64(data, rows, cols, X, "Q6_K")
    for prec in ("auto", "fp32"):
        err = normalized_error(QuantMatrix(data, "Q6_K", rows, cols).matmul_t(X, precision=prec),
                               want, norms, X)
        assert err < FP32_TOL, (prec, err)


def test_exact_fp16_q6k_bits_do_not_depend_on_m():
    rows, cols = 700, 4096
    data = synth.random_matrix_bytes("Q6_K", rows, cols, seed=19)
    qm = QuantMatrix(data, "Q6_K", rows, cols)
    X = synth.random_x(cols, seed=20, batch=150)
    whole = qm.matmul_t(X, precision="fp32")
    parts = np.concatenate([qm.matmul_t(X[a:b], precision="fp32")
                            for a, b in ((0, 7), (7, 71), (71, 150))])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))


def test_exact_fp16_q6k_x_rows():
    """Rows of zeros, of 1e30, of 1e-30, of 1e-20 beside 1e20, and a NaN and
    an infinity, which make only their own rows non-finite."""
    rows, cols, M = 512, 2048, 72
    data = synth.random_matrix_bytes("Q6_K", rows, cols, seed=23)
    X = synth.random_x(cols, seed=24, batch=M)
    X[0] = 0
    X[1] *= 1e30
    X[2] *= 1e-30
    X[3, ::2] *= 1e-20
    X[3, 1::2] *= 1e20
    X[5, 100] = np.nan
    X[6, 7] = np.inf
    Y = QuantMatrix(data, "Q6_K", rows, cols).matmul_t(X, precision="fp32")
    assert np.all(Y[0] == 0)
    assert not np.isfinite(Y[5]).any() and not np.isfinite(Y[6]).any()
    keep = [i for i in range(M) if i not in (5, 6)]
    want, norms = _f64(data, rows, cols, X[keep], "Q6_K")
    assert normalized_error(Y[keep], want, norms, X[keep]) < FP32_TOL


# ---- Q5_K: the Q4_K kernel with the fifth code bit (sc*code <= 1953) --------

def _adversarial_q5k(rows, cols, seed):
    """Random bytes everywhere; d and dmin finite fp16 of either sign."""
    nb = rows * cols // 256
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, 176), dtype=np.uint8)
    for o in (0, 2):
        mag = 10.0 ** rng.uniform(-7.5, 0.5, nb)
        b[:, o:o + 2] = (mag * rng.choice([-1.0, 1.0], nb)).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b.tobytes()


@pytest.mark.parametrize("layout", ["raw", "split"])
@pytest.mark.parametrize("precision", ["auto", "fp32"])
@pytest.mark.parametrize("M,rows,cols", [(8, 512, 2048), (16, 4096, 4096), (37, 1000, 2048),
                                         (130, 700, 4096), (513, 256, 2048), (64, 1024, 14336)])
def test_exact_fp16_q5k_vs_f64(M, rows, cols, precision, layout):
    data = synth.random_matrix_bytes("Q5_K", rows, cols, seed=rows + M)
    X = synth.random_x(cols, seed=M, batch=M)
    qm = QuantMatrix(data, "Q5_K", rows, cols, layout=layout)
    want, norms = _f64(data, rows, cols, X, "Q5_K")
    err = normalized_error(qm.matmul_t(X, precision=precision), want, norms, X)
    assert err < FP32_TOL, err


@pytest.mark.parametrize("M", [8, 16, 100])
def test_exact_fp16_q5k_adversarial_blocks(M):
    rows, cols = 384, 2048
    data = _adversarial_q5k(rows, cols, seed=M)
    X = synth.random_x(cols, seed=M + 1, batch=M)
    want, norms = _f64(data, rows, cols, X, "Q5_K")
    for prec in ("auto", "fp32"):
        err = normalized_error(QuantMatrix(data, "Q5_K", rows, cols).matmul_t(X, precision=prec),
                               want, norms, X)
        assert err < FP32_TOL, (prec, err)


def test_exact_fp16_q5k_fused_x_and_m_invariance():
    rows, cols = 1000, 4096
    data = synth.random_matrix_bytes("Q5_K", rows, cols, seed=29)
    qm = QuantMatrix(data, "Q5_K", rows, cols)
    X = synth.random_x(cols, seed=30, batch=150)
    prepared = _with_env("AQ_MATMUL_X_PREP", lambda: qm.matmul_t(X[:16]))
    assert np.array_equal(qm.matmul_t(X[:16]).view(np.uint32), prepared.view(np.uint32))
    whole = qm.matmul_t(X, precision="fp32")
    parts = np.concatenate([qm.matmul_t(X[a:b], precision="fp32")
                            for a, b in ((0, 7), (7, 71), (71, 150))])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))


# ---- per-32 block formats: one 16x16x32 product per block, d per block ------

B32 = {"Q8_0": (34, (0,)), "Q4_0": (18, (0,)), "Q4_1": (20, (0, 2)), "Q5_0": (22, (0,)),
       "Q5_1": (24, (0, 2))}  # block bytes, offsets of the fp16 d (and m) fields


def _adversarial_b32(dtype, rows, cols, seed):
    """Random bytes everywhere; d (and m) finite fp16 of either sign."""
    bb, fields = B32[dtype]
    nb = rows * cols // 32
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    for o in fields:
        mag = 10.0 ** rng.uniform(-7.5, 0.5, nb)
        b[:, o:o + 2] = (mag * rng.choice([-1.0, 1.0], nb)).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b.tobytes()


@pytest.mark.parametrize("dtype", list(B32))
@pytest.mark.parametrize("precision", ["auto", "fp32"])
@pytest.mark.parametrize("M,rows,cols", [(64, 300, 2048), (130, 1000, 4096), (513, 256, 2048),
                                         (70, 2048, 14336)])
def test_exact_fp16_b32_vs_f64(dtype, M, rows, cols, precision):
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=rows + M)
    X = synth.random_x(cols, seed=M, batch=M)
    want, norms = _f64(data, rows, cols, X, dtype)
    err = normalized_error(QuantMatrix(data, dtype, rows, cols).matmul_t(X, precision=precision),
                           want, norms, X)
    assert err < FP32_TOL, err


@pytest.mark.parametrize("dtype", list(B32))
def test_exact_fp16_b32_adversarial_and_m_invariance(dtype):
    rows, cols = 384, 2048
    data = _adversarial_b32(dtype, rows, cols, seed=len(dtype))
    qm = QuantMatrix(data, dtype, rows, cols)
    X = synth.random_x(cols, seed=41, batch=150)
    X[3] *= 1e-30
    X[4, ::2] *= 1e20
    want, norms = _f64(data, rows, cols, X, dtype)
    whole = qm.matmul_t(X, precision="fp32")
    assert normalized_error(whole, want, norms, X) < FP32_TOL
    assert normalized_error(qm.matmul_t(X), want, norms, X) < FP32_TOL
    parts = np.concatenate([qm.matmul_t(X[a:b], precision="fp32")
                            for a, b in ((0, 7), (7, 71), (71, 150))])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))


@pytest.mark.parametrize("dtype", ["Q8_0", "Q5_1"])
def test_exact_fp16_b32_k_not_multiple_of_256(dtype):
    """K = 4128 (129 blocks): not whole 256-column groups, so the fp32 MFMA
    path serves it, to the same bar."""
    rows, cols, M = 300, 4128, 70
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=43)
    X = synth.random_x(cols, seed=44, batch=M)
    want, norms = _f64(data, rows, cols, X, dtype)
    for prec in ("auto", "fp32"):
        err = normalized_error(QuantMatrix(data, dtype, rows, cols).matmul_t(X, precision=prec),
                               want, norms, X)
        assert err < FP32_TOL, (prec, err)


@pytest.mark.parametrize("dtype", ["Q4_K", "Q5_K", "Q6_K"] + list(B32))
@pytest.mark.parametrize("M", [1, 17, 64])
def test_exact_fp16_smallest_k_and_ragged_rows(dtype, M):
    """K = 256 (one super-block, or one group of 8 blocks of 32) and 17 rows:
    one partial tile in every direction, at both precisions (fp32 takes the
    exact kernels at any M)."""
    rows, cols = 17, 256
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M + 50)
    X = synth.random_x(cols, seed=M + 51, batch=M)
    want, norms = _f64(data, rows, cols, X, dtype)
    qm = QuantMatrix(data, dtype, rows, cols)
    for prec in ("auto", "fp32"):
        err = normalized_error(qm.matmul_t(X, precision=prec), want, norms, X)
        assert err < FP32_TOL, (prec, err)


@pytest.mark.parametrize("dtype", ["Q6_K"] + list(B32))
@pytest.mark.parametrize("M", [9, 16, 24, 40])
def test_exact_fp16_small_tiles(dtype, M):
    """The small batches' tiles of the Q6_K and per-32 kernels (16 x 128 up
    to 16 rows, 32 x 256 (Q6_K 32 x 128) up to 32, 64 x 256 above): split
    over workgroups at the default precision, unsplit at fp32, both within
    the float32 bar, and the unsplit outputs bit-identical to the same rows
    in a 64-row launch (the same arithmetic per output in every shape)."""
    print(f"exact small tiles {dtype} M={M}", flush=True)
    rows, cols = 1000, 4096
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M + 60)
    X = synth.random_x(cols, seed=M + 61, batch=64)
    qm = QuantMatrix(data, dtype, rows, cols)
    want, norms = _f64(data, rows, cols, X[:M], dtype)
    for prec in ("auto", "fp32"):
        err = normalized_error(qm.matmul_t(X[:M], precision=prec), want, norms, X[:M])
        assert err < FP32_TOL, (prec, err)
    small = qm.matmul_t(X[:M], precision="fp32")
    whole = qm.matmul_t(X, precision="fp32")
    assert np.array_equal(small.view(np.uint32), whole[:M].view(np.uint32))


# ---- the batched step's gate/up product with the SwiGLU in one call -------

@pytest.mark.parametrize("dtype", ["Q4_K", "Q5_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("precision", ["fp32", "auto"])
@pytest.mark.parametrize("M", [16, 64, 513])
def test_matmul_t_swiglu_matches_separate_calls(dtype, precision, M):
    """aq_matmul_t_swiglu against aq_matmul_t then aq_swiglu_pairs, bit for
    bit: Q4_K and Q5_K form the pairs in the exact kernel's store where it
    runs unsplit, the others (and split launches) go through the scratch
    product and the pairs kernel."""
    import ctypes

    import torch

    from alpacca_amd import _lib
    rows, cols = 1024, 2048
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M + 61)
    qm = QuantMatrix(data, dtype, rows, cols)
    dev = torch.device("cuda", 0)
    X = torch.from_numpy(synth.random_x(cols, seed=M + 62, batch=M)).to(dev)
    Z = torch.empty((M, rows), dtype=torch.float32, device=dev)
    want = torch.empty((M, rows // 2), dtype=torch.float32, device=dev)
    got = torch.full((M, rows // 2), float("nan"), dtype=torch.float32, device=dev)
    qm.matmul_t_device(X.data_ptr(), M, Z.data_ptr(), 0, precision)
    _lib.check(_lib.load().aq_swiglu_pairs(ctypes.c_void_p(Z.data_ptr()), M * rows // 2,
                                           ctypes.c_void_p(want.data_ptr()), None))
    Z.fill_(float("nan"))
    qm.matmul_t_swiglu_device(X.data_ptr(), M, Z.data_ptr(), got.data_ptr(), 0, precision)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_matmul_t_swiglu_rejects_odd_rows_and_host_pointers():
    import ctypes

    from alpacca_amd import _lib
    qm = QuantMatrix(synth.random_matrix_bytes("Q4_K", 3, 256, seed=1), "Q4_K", 3, 256)
    lib = _lib.load()
    rc = lib.aq_matmul_t_swiglu(ctypes.c_void_p(qm._handle), None, 0, None, None, 0,
                                _lib.AQ_IN_DEVICE | _lib.AQ_OUT_DEVICE, None)
    assert rc == _lib.AQ_ERR_VALUE
    qm2 = QuantMatrix(synth.random_matrix_bytes("Q4_K", 4, 256, seed=1), "Q4_K", 4, 256)
    assert lib.aq_matmul_t_swiglu(ctypes.c_void_p(qm2._handle), None, 0, None, None, 0, 0,
                                  None) == _lib.AQ_ERR_VALUE


@pytest.mark.parametrize("dtype", ["Q4_K", "Q5_K"])
def test_exact_fp16_fused_x_unsplit_is_m_invariant(dtype):
    """At K = 1024 a chunk of up to 16 rows runs the fused X staging without
    a split (its per-split scale is then the whole row's), larger chunks the
    prepared pieces: fp32 precision still gives the rows of the whole
    product bit for bit."""
    rows, cols = 700, 1024
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=71)
    qm = QuantMatrix(data, dtype, rows, cols)
    X = synth.random_x(cols, seed=72, batch=150)
    whole = qm.matmul_t(X, precision="fp32")
    parts = np.concatenate([qm.matmul_t(X[a:b], precision="fp32")
                            for a, b in ((0, 7), (7, 23), (23, 39), (39, 150))])
    assert np.array_equal(whole.view(np.uint32), parts.view(np.uint32))
