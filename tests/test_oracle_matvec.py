"""Pins the matvec / matmul_t oracle (oracle/qmatrix_ref.py) and the CPU
baseline transliteration: closed-form special cases, brute force on tiny
inputs, the reference's own differential checks and tolerances
(tests/smoke.py:165-177, :275-300, :318-358)."""
from __future__ import annotations

import numpy as np
import pytest

from alpacca_amd import synth
from oracle import quants_ref as Q
from oracle.qmatrix_ref import RefMatrix, normalized_error
from tests import smoke_patterns as SP

FORMATS = list(Q.GEOMETRY)


def small(dtype, rows=6, seed=0):
    be = Q.GEOMETRY[dtype][0]
    cols = 2 * be if be == 256 else 4 * be
    return synth.random_matrix_bytes(dtype, rows, cols, seed), rows, cols


@pytest.mark.parametrize("dtype", FORMATS)
def test_unit_vectors_give_columns_and_ones_give_row_sums(dtype):
    data, rows, cols = small(dtype)
    ref = RefMatrix(data, dtype, rows, cols)
    W = ref.dense().astype(np.float64)
    for k in (0, cols // 3, cols - 1):
        e = np.zeros(cols)
        e[k] = 1.0
        assert np.array_equal(ref.matvec_f64(e), W[:, k])
    assert np.allclose(ref.matvec_f64(np.ones(cols)), W.sum(axis=1), rtol=0, atol=1e-12)


@pytest.mark.parametrize("dtype", FORMATS)
def test_f64_matvec_equals_brute_force_loops(dtype):
    data, rows, cols = small(dtype, rows=3)
    ref = RefMatrix(data, dtype, rows, cols)
    W = Q.exact_decode(data, dtype).reshape(rows, cols)
    x = synth.random_x(cols, seed=9).astype(np.float64)
    brute = [sum(float(W[r, c]) * float(x[c]) for c in range(cols)) for r in range(rows)]
    assert np.allclose(ref.matvec_f64(x), brute, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype", FORMATS)
def test_matvec_is_linear(dtype):
    data, rows, cols = small(dtype)
    ref = RefMatrix(data, dtype, rows, cols)
    a, b = synth.random_x(cols, 1).astype(np.float64), synth.random_x(cols, 2).astype(np.float64)
    lhs = ref.matvec_f64(2.5 * a - 0.75 * b)
    rhs = 2.5 * ref.matvec_f64(a) - 0.75 * ref.matvec_f64(b)
    assert normalized_error(lhs, rhs, ref.row_norms(), np.abs(a) + np.abs(b)) < 1e-12


@pytest.mark.parametrize("fmt,rows,cols", SP.SMALL_CASES + SP.LARGE_CASES)
def test_reference_order_matvec_and_matmul(fmt, rows, cols):
    """The float32 restatement of QuantMatrix.matvec (both of its branches:
    small batched-matmul and >= 2**20-element einsum) and matmul_t against the
    reference's own bars, and within 2e-5 of the float64 anchor."""
    data = SP.packed(fmt, rows, cols, Q.quantize_q8_0, Q.quantize_q4_0)
    ref = RefMatrix(data, fmt, rows, cols)
    x = np.asarray(SP.x_vector(cols), dtype=np.float32)
    y = ref.matvec_ref(x)
    assert float(np.max(np.abs(y - ref.dense() @ x))) < 1e-3
    assert normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x) < 2e-5
    X = np.stack([x, x * 0.5 - 0.1]).astype(np.float32)
    Y = ref.matmul_t_ref(X)
    stacked = np.stack([ref.matvec_ref(r) for r in X])
    assert float(np.max(np.abs(Y - stacked))) < 1e-3
    assert normalized_error(Y, ref.matmul_t_f64(X), ref.row_norms(), X) < 2e-5
    idx = [0, rows - 1, min(1, rows - 1)]
    assert np.array_equal(ref.rows_at(idx), ref.dense()[idx])


def test_large_q8_0_branch():
    """smoke.py:320-336: 4096x288 Q8_0 takes the einsum branch."""
    rows, cols = 4096, 288
    vals = [((i * 37) % 251) / 251.0 - 0.5 for i in range(rows * cols)]
    data = Q.quantize_q8_0(vals)
    ref = RefMatrix(data, "Q8_0", rows, cols)
    assert rows * cols >= 1 << 20
    x = np.asarray([((i * 19) % 67) / 23.0 - 1.4 for i in range(cols)], dtype=np.float32)
    assert float(np.max(np.abs(ref.matvec_ref(x) - ref.dense() @ x))) < 1e-3


def test_normalized_error_definition():
    norms = np.array([2.0, 4.0])
    x = np.array([3.0, 4.0])  # ||x|| = 5
    assert normalized_error([1.0, 1.0], [0.0, 0.0], norms, x) == pytest.approx(0.1)
    X = np.array([[3.0, 4.0], [6.0, 8.0]])
    err = normalized_error([[0.0, 0.0], [0.0, 2.0]], np.zeros((2, 2)), norms, X)
    assert err == pytest.approx(2.0 / (10.0 * 4.0))


def test_cpu_baseline_transliteration_matches():
    """The C/OpenMP transliteration of the reference's Numba loop
    (alpacca/kernels.py:49-69) computes the same product."""
    from oracle import cbaseline
    if not any((cbaseline.BUILD / f).exists() for f in
               ("libmatvec_loop_v3.so", "libmatvec_loop_v4.so")):
        cbaseline.build()
    for dtype in ("Q4_K", "Q6_K", "Q8_0", "Q5_1"):
        data, rows, cols = small(dtype, rows=64, seed=4)
        ref = RefMatrix(data, dtype, rows, cols)
        x = synth.random_x(cols, seed=5)
        y = cbaseline.LoopMatvec(ref.q3, ref.d, ref.m)(x)
        assert normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x) < 2e-5


def test_int8_activation_scheme_identities():
    """quantize_x_q8: round trip within d/2, all-zero blocks give zero, the
    largest element maps to +-127; matmul_t_int8_f64 equals the float64
    product of the dequantized operands."""
    from oracle.qmatrix_ref import RefMatrix, quantize_x_q8
    rng = np.random.default_rng(8)
    X = rng.standard_normal((7, 128)).astype(np.float32)
    X[2, 32:64] = 0.0
    q, d = quantize_x_q8(X)
    deq = (q.reshape(7, 4, 32).astype(np.float64) * d[:, :, None]).reshape(7, 128)
    assert np.all(np.abs(deq - X) <= d.repeat(32, axis=1) / 2 * (1 + 1e-6))
    assert np.all(q[2, 32:64] == 0) and d[2, 1] == 0
    assert np.all(np.abs(q).reshape(7, 4, 32).max(axis=2)[d > 0] == 127)
    data = synth.random_matrix_bytes("Q8_0", 5, 128, seed=3)
    ref = RefMatrix(data, "Q8_0", 5, 128)
    assert np.allclose(ref.matmul_t_int8_f64(X), deq @ ref.dense().astype(np.float64).T,
                       rtol=1e-12, atol=1e-12)
