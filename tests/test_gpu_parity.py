"""Parity of the HIP path (through the C ABI) with the CPU oracle.

Bars:
* decoded weights (row gather) bit-identical to the reference decoder;
* matvec and fp32 matmul_t within 2e-5 of the float64 oracle, normalized
  per output by ||W_r|| * ||x||;
* bf16 MFMA matmul_t within 1e-2 under the same normalization.
"""
from __future__ import annotations

import numpy as np
import pytest

from alpacca_amd import synth
from alpacca_amd.qmatrix import QuantMatrix
from oracle import quants_ref as Q
from oracle.qmatrix_ref import RefMatrix, normalized_error
from tests import smoke_patterns as SP

pytestmark = pytest.mark.gpu

FP32_TOL = 2e-5
BF16_TOL = 1e-2
FORMATS = ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q4_0", "Q4_1", "Q5_0", "Q5_1"]
LAYOUTS = {"Q4_K": ["raw", "split"], "Q5_K": ["raw", "split"]}
FMT_LAYOUTS = [(f, lay) for f in FORMATS for lay in LAYOUTS.get(f, ["split"])]


def _adversarial_blocks(dtype, nblocks, seed):
    """Uniform random bytes everywhere, fp16 fields finite but of either sign
    and spanning normal and subnormal magnitudes."""
    be, bb, _, _ = Q.GEOMETRY[dtype]
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(nblocks, bb), dtype=np.uint8)
    offs = {"Q6_K": [208], "Q4_K": [0, 2], "Q5_K": [0, 2], "Q4_1": [0, 2],
            "Q5_1": [0, 2]}.get(dtype, [0])
    for o in offs:
        mag = 10.0 ** rng.uniform(-7.5, 0.5, nblocks)
        sign = rng.choice([-1.0, 1.0], nblocks)
        b[:, o:o + 2] = (mag * sign).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b


def _chunked_f64(data, dtype, rows, cols, x, chunk=4096):
    """float64 W @ x and the row norms, decoding W a few thousand rows at a time."""
    be, bb, _, _ = Q.GEOMETRY[dtype]
    row_bytes = cols // be * bb
    raw = np.frombuffer(data, dtype=np.uint8)
    y = np.empty(rows)
    norms = np.empty(rows)
    x64 = np.asarray(x, dtype=np.float64)
    for r0 in range(0, rows, chunk):
        r1 = min(rows, r0 + chunk)
        W = Q.dequantize(raw[r0 * row_bytes:r1 * row_bytes], (r1 - r0) * cols,
                         dtype).reshape(r1 - r0, cols).astype(np.float64)
        y[r0:r1] = W @ x64
        norms[r0:r1] = np.linalg.norm(W, axis=1)
    return y, norms


# ---------------------------------------------------------------- decode ---

@pytest.mark.parametrize("dtype,layout", FMT_LAYOUTS)
def test_rows_bit_exact_adversarial(dtype, layout):
    be = Q.GEOMETRY[dtype][0]
    rows, cols = 37, 3 * be
    data = _adversarial_blocks(dtype, rows * 3, seed=11).tobytes()
    qm = QuantMatrix(data, dtype, rows, cols, layout=layout)
    assert qm.layout == layout
    got = qm.rows_at(np.arange(rows))
    ref = Q.dequantize(data, rows * cols, dtype).reshape(rows, cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # gather order, repeats and single-row access
    idx = [rows - 1, 0, 5, 5]
    assert np.array_equal(qm.rows_at(idx).view(np.uint32), ref[idx].view(np.uint32))
    assert np.array_equal(qm.row(3).view(np.uint32), ref[3].view(np.uint32))


@pytest.mark.parametrize("dtype", FORMATS)
def test_rows_bit_exact_config_blocks(dtype):
    rows, cols = 300, 2048
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=5)
    qm = QuantMatrix(data, dtype, rows, cols)
    ref = Q.dequantize(data, rows * cols, dtype).reshape(rows, cols)
    got = qm.rows_at(np.arange(rows))
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


# -------------------------------------------------- reference smoke cases ---

@pytest.mark.parametrize("fmt,rows,cols", SP.SMALL_CASES + SP.LARGE_CASES)
def test_reference_smoke_cases(fmt, rows, cols):
    """smoke.py:134-358 on the HIP path: decode equals the decoder, matvec
    matches dense (< 1e-3, the reference's bar, and our 2e-5 normalized),
    matmul_t matches stacked matvecs, row lookups match, bad rows raise."""
    packed = SP.packed(fmt, rows, cols, Q.quantize_q8_0, Q.quantize_q4_0)
    qm = QuantMatrix(packed, fmt, rows, cols)
    ref = RefMatrix(packed, fmt, rows, cols)
    dense = ref.dense()
    x = np.asarray(SP.x_vector(cols), dtype=np.float32)
    y = qm.matvec(x)
    assert float(np.max(np.abs(y - dense @ x))) < 1e-3
    assert normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x) < FP32_TOL
    X = np.stack([x, x * 0.5 - 0.1]).astype(np.float32)
    stacked = np.stack([qm.matvec(r) for r in X])
    assert float(np.max(np.abs(qm.matmul_t(X) - stacked))) < 1e-3
    r = min(3, rows - 1)
    assert np.array_equal(qm.row(r), dense[r])
    idx = [0, rows - 1, min(1, rows - 1)]
    assert np.array_equal(qm.rows_at(idx), dense[idx])
    with pytest.raises(IndexError):
        qm.rows_at([rows])
    with pytest.raises(IndexError):
        qm.rows_at([-1])
    with pytest.raises(IndexError):
        qm.row(rows)
    assert qm.data is None
    assert qm.storage_nbytes() * 3 <= rows * cols * 4 + 4096


@pytest.mark.parametrize("fmt,layout", [("Q4_K", "raw"), ("Q4_K", "split"), ("Q6_K", "split"),
                                        ("Q8_0", "split"), ("Q5_K", "raw")])
def test_storage_nbytes_is_the_device_allocation(fmt, layout):
    # raw: exactly the GGUF bytes; split: every plane padded to 256 bytes, so
    # the allocation is a multiple of 256 and exceeds the blocks by less than
    # 256 bytes per plane (at most four planes)
    rows, cols = 37, 512
    raw = synth.random_matrix_bytes(fmt, rows, cols, seed=5)
    qm = QuantMatrix(raw, fmt, rows, cols, layout=layout)
    assert qm.layout == layout
    n = qm.storage_nbytes()
    if layout == "raw":
        assert n == len(raw)
    else:
        assert n % 256 == 0 and len(raw) <= n < len(raw) + 4 * 256


# ---------------------------------------------------------------- matvec ---

MATVEC_CASES = [
    ("Q8_0", 2048, 2048),                     # config 1
    ("Q4_K", 2048, 2048), ("Q4_K", 512, 2048),
    ("Q4_K", 8192, 2048), ("Q4_K", 2048, 8192),   # config 2 (1B shapes)
    ("Q4_K", 4096, 4096), ("Q4_K", 1024, 4096),
    ("Q4_K", 14336, 4096), ("Q4_K", 4096, 14336),  # the metric's 8B shapes
    ("Q5_K", 4096, 4096), ("Q5_K", 1024, 4096), ("Q5_K", 14336, 4096),  # config 3
    ("Q6_K", 4096, 14336), ("Q6_K", 128256, 4096),
    ("Q4_0", 4096, 4096), ("Q4_1", 1024, 4096), ("Q5_0", 1024, 4096),
    ("Q5_1", 1024, 4096),
    ("Q4_K", 7, 256), ("Q6_K", 1, 256), ("Q8_0", 3, 32),   # tiny / ragged
    ("Q4_K", 1000, 2304), ("Q8_0", 999, 4000),
]


@pytest.mark.parametrize("dtype,rows,cols", MATVEC_CASES)
def test_matvec_vs_f64(dtype, rows, cols):
    print(f"matvec {dtype} {rows}x{cols}", flush=True)
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=rows + cols)
    x = synth.random_x(cols, seed=3)
    qm = QuantMatrix(data, dtype, rows, cols)
    ref, norms = _chunked_f64(data, dtype, rows, cols, x)
    for kernel in ("int8", "fp32"):
        y = qm.matvec(x, kernel=kernel)
        err = normalized_error(y, ref, norms, x)
        assert err < FP32_TOL, (kernel, err)
        # deterministic: same call, same bits
        assert np.array_equal(qm.matvec(x, kernel=kernel), y)


@pytest.mark.parametrize("dtype", FORMATS)
def test_matvec_int8_x_edge_cases(dtype):
    """x groups that are all zero, single spikes, huge/tiny magnitudes and
    exact ties of the piece rounding - the int8 split must stay in bounds."""
    be = Q.GEOMETRY[dtype][0]
    rows, cols = 64, 8 * max(be, 64)
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=21)
    qm = QuantMatrix(data, dtype, rows, cols)
    ref = RefMatrix(data, dtype, rows, cols)
    rng = np.random.default_rng(5)
    xs = [np.zeros(cols, np.float32),
          np.where(np.arange(cols) % 97 == 3, 1e30, 0).astype(np.float32),
          (rng.standard_normal(cols) * 1e-30).astype(np.float32),
          (rng.standard_normal(cols) * 1e30).astype(np.float32),
          (np.arange(cols) % 255 - 127).astype(np.float32) / 127.0,
          np.repeat(rng.standard_normal(cols // 32), 32).astype(np.float32),
          (rng.standard_normal(cols) * 1e-39).astype(np.float32),   # subnormal
          np.where(np.arange(cols) % 33 == 0, 1e36, -1e-20).astype(np.float32)]
    x = rng.standard_normal(cols).astype(np.float32)
    x[: cols // 2] = 0.0
    xs.append(x)
    for x in xs:
        y = qm.matvec(x)
        err = normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x)
        assert err < FP32_TOL, err


@pytest.mark.parametrize("dtype", ["Q4_K", "Q6_K", "Q8_0", "Q4_0"])
def test_matvec_nonfinite_x_propagates(dtype):
    """A NaN or infinity in x makes every output non-finite, as the float
    product does (rows whose weights in that column are 0 give 0 * inf =
    NaN in the reference too)."""
    be = Q.GEOMETRY[dtype][0]
    rows, cols = 16, 4 * max(be, 64)
    qm = QuantMatrix(synth.random_matrix_bytes(dtype, rows, cols, seed=22), dtype, rows, cols)
    for bad in (np.nan, np.inf, -np.inf):
        x = synth.random_x(cols, seed=6)
        x[cols // 3] = bad
        for kernel in ("int8", "fp32"):
            assert not np.isfinite(qm.matvec(x, kernel=kernel)).any(), (bad, kernel)


@pytest.mark.parametrize("dtype,layout", FMT_LAYOUTS)
def test_matvec_layouts_and_adversarial(dtype, layout):
    be = Q.GEOMETRY[dtype][0]
    rows, cols = 333, 24 * be if be == 32 else 9 * be
    data = _adversarial_blocks(dtype, rows * (cols // be), seed=7).tobytes()
    x = synth.random_x(cols, seed=4)
    qm = QuantMatrix(data, dtype, rows, cols, layout=layout)
    ref = RefMatrix(data, dtype, rows, cols)
    err = normalized_error(qm.matvec(x), ref.matvec_f64(x), ref.row_norms(), x)
    assert err < FP32_TOL, err


@pytest.mark.parametrize("dtype", ["Q4_K", "Q6_K", "Q8_0", "Q5_1"])
def test_matvec_unit_vector_is_column(dtype):
    """x = e_k selects column k of the decoded matrix.  In the fp32 kernel
    every partial product is exact, so the result must equal the decoded
    column bit-for-bit; the int8 kernel (x = 127 * (1/127)) within 2e-5."""
    rows, cols = 4096, 4096
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=9)
    qm = QuantMatrix(data, dtype, rows, cols)
    rng = np.random.default_rng(0)
    for k in rng.integers(0, cols, 3):
        x = np.zeros(cols, np.float32)
        x[k] = 1.0
        W = Q.dequantize(data, rows * cols, dtype).reshape(rows, cols)
        ref = W[:, k]
        assert np.array_equal(qm.matvec(x, kernel="fp32"), ref)
        norms = np.linalg.norm(W.astype(np.float64), axis=1)
        assert normalized_error(qm.matvec(x, kernel="int8"), ref, norms, x) < FP32_TOL


def test_matvec_reference_order_agrees():
    """Our result and the reference's own float32 order sit within the same
    normalized bound of the float64 anchor."""
    rows, cols = 4096, 4096
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=2)
    x = synth.random_x(cols, seed=8)
    ref = RefMatrix(data, "Q4_K", rows, cols)
    anchor, norms = ref.matvec_f64(x), ref.row_norms()
    assert normalized_error(ref.matvec_ref(x), anchor, norms, x) < FP32_TOL
    assert normalized_error(QuantMatrix(data, "Q4_K", rows, cols).matvec(x),
                            anchor, norms, x) < FP32_TOL


def test_matvec_device_pointers():
    torch = pytest.importorskip("torch")
    rows, cols = 2048, 2048
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=1)
    x = synth.random_x(cols, seed=2)
    qm = QuantMatrix(data, "Q4_K", rows, cols)
    yd = qm.matvec(torch.from_numpy(x).cuda())
    assert yd.is_cuda
    assert np.array_equal(yd.cpu().numpy(), qm.matvec(x))


# -------------------------------------------------------------- matmul_t ---

MATMUL_CASES = [
    ("Q4_K", 512, 14336, 4096), ("Q4_K", 512, 4096, 14336),   # config 4
    ("Q8_0", 512, 4096, 4096),
    ("Q6_K", 256, 2048, 8192), ("Q5_K", 130, 1024, 4096),
    ("Q4_0", 64, 999, 96), ("Q4_1", 65, 256, 64), ("Q5_0", 200, 130, 32),
    ("Q5_1", 3, 77, 160), ("Q4_K", 1, 300, 512),
]


@pytest.mark.parametrize("dtype,M,rows,cols", MATMUL_CASES)
@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_matmul_t_vs_f64(dtype, M, rows, cols, precision):
    print(f"matmul_t {dtype} M={M} {rows}x{cols} {precision}", flush=True)
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M + rows)
    X = synth.random_x(cols, seed=6, batch=M)
    qm = QuantMatrix(data, dtype, rows, cols)
    Y = qm.matmul_t(X, precision=precision)
    assert Y.shape == (M, rows)
    # check a subset of W rows against float64 (all rows for small cases)
    rng = np.random.default_rng(1)
    sel = np.sort(rng.choice(rows, size=min(rows, 512), replace=False))
    W = qm.rows_at(sel).astype(np.float64)  # bit-exact decode (tested above)
    ref = X.astype(np.float64) @ W.T
    err = normalized_error(Y[:, sel], ref, np.linalg.norm(W, axis=1), X)
    assert err < (FP32_TOL if precision == "fp32" else BF16_TOL), err


SMALL_BATCH_CASES = [
    ("Q4_K", 4096, 4096), ("Q4_K", 512, 2048), ("Q6_K", 300, 14336), ("Q5_K", 200, 4096),
    ("Q8_0", 256, 2048), ("Q4_0", 130, 1024), ("Q5_1", 70, 4096),
]


@pytest.mark.parametrize("M", [2, 3, 5, 8, 16, 63])
@pytest.mark.parametrize("dtype,rows,cols", SMALL_BATCH_CASES)
def test_matmul_t_small_batch(dtype, rows, cols, M):
    """Batches below 64 rows (the short suffixes of model.py:618-637): 2
    rows of Q4_K / Q5_K and up to 4 of Q6_K and the per-32 formats run the
    integer decode kernel with the x vectors sharing one weight
    stream, more rows the exact fp16 kernels' small tiles (ragged here): within
    the matvec bar (2e-5 of ||W_r||*||x||) of the float64 product, every row
    of Y its own x's product, including rows wider than a pass of staged
    vectors (column windows) and row pairs (K <= 2048)."""
    print(f"matmul_t small batch {dtype} M={M} {rows}x{cols}", flush=True)
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M * 7 + rows)
    X = synth.random_x(cols, seed=M + 3, batch=M)
    qm, ref = QuantMatrix(data, dtype, rows, cols), RefMatrix(data, dtype, rows, cols)
    Y = qm.matmul_t(X)
    assert Y.shape == (M, rows)
    want = ref.matmul_t_f64(X)
    assert normalized_error(Y, want, ref.row_norms(), X) < FP32_TOL
    # the vectors are independent: row v is X[v]'s own product
    for v in (0, M - 1):
        assert normalized_error(Y[v], want[v], ref.row_norms(), X[v]) < FP32_TOL


def test_matmul_t_small_batch_device_pointers():
    """The device form enqueues on the caller's stream and writes only its
    M x rows block of Y."""
    torch = pytest.importorskip("torch")
    rows, cols, M = 1000, 4096, 5
    data = synth.random_matrix_bytes("Q4_K", rows, cols, seed=31)
    X = synth.random_x(cols, seed=32, batch=M)
    qm, ref = QuantMatrix(data, "Q4_K", rows, cols), RefMatrix(data, "Q4_K", rows, cols)
    Xd = torch.from_numpy(X).cuda()
    Yd = torch.full((M + 1, rows), 7.0, device="cuda")
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        qm.matmul_t_device(Xd.data_ptr(), M, Yd.data_ptr(), s.cuda_stream)
    s.synchronize()
    Y = Yd.cpu().numpy()
    assert np.all(Y[M] == 7.0)
    assert normalized_error(Y[:M], ref.matmul_t_f64(X), ref.row_norms(), X) < FP32_TOL


def test_matmul_t_fp32_equals_stacked_matvec():
    rows, cols = 1000, 2048
    data = synth.random_matrix_bytes("Q6_K", rows, cols, seed=12)
    X = synth.random_x(cols, seed=13, batch=5)
    qm = QuantMatrix(data, "Q6_K", rows, cols)
    Y = qm.matmul_t(X)  # M < 64: fp32
    ref = RefMatrix(data, "Q6_K", rows, cols)
    for m in range(5):
        assert normalized_error(Y[m], qm.matvec(X[m]), ref.row_norms(), X[m]) < FP32_TOL


# ------------------------------------------------------------ error paths ---

def test_error_classes_on_device():
    data = synth.random_matrix_bytes("Q4_K", 4, 256, seed=0)
    qm = QuantMatrix(data, "Q4_K", 4, 256)
    with pytest.raises(ValueError):
        qm.matvec(np.zeros(255, np.float32))
    with pytest.raises(ValueError):
        qm.matmul_t(np.zeros((2, 255), np.float32))
    with pytest.raises(ValueError):
        qm.matmul_t(np.zeros(256, np.float32))
    with pytest.raises(IndexError):
        qm.row(-1)
    with pytest.raises(IndexError):
        qm.rows_at([0, 4])
    assert qm.rows_at([]).shape == (0, 256)
    assert qm.matmul_t(np.zeros((0, 256), np.float32)).shape == (0, 4)
    with pytest.raises(ValueError):
        QuantMatrix(data, "Q6_K", 4, 256, layout="raw")


# ------------------------------------------------- kernel configurations ---

CFG_CASES = [("Q4_K", 1000, 4096), ("Q4_K", 777, 14336), ("Q6_K", 300, 2048),
             ("Q8_0", 513, 4096), ("Q5_K", 64, 8192), ("Q4_0", 100, 2048)]


@pytest.mark.parametrize("dtype,rows,cols", CFG_CASES)
def test_matvec_every_config(dtype, rows, cols, monkeypatch):
    """Every rows-in-flight setting (RC) and workgroup size (WG) of the
    integer kernel and any wave budget (waves per CU) give the same answer
    within tolerance; invalid settings fall back to the defaults."""
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=31)
    x = synth.random_x(cols, seed=32)
    qm = QuantMatrix(data, dtype, rows, cols)
    ref = RefMatrix(data, dtype, rows, cols)
    anchor, norms = ref.matvec_f64(x), ref.row_norms()
    for wpc in ["0", "1", "3", "64"]:
        monkeypatch.setenv("AQ_MATVEC_WPC", wpc)
        for rc in ["1", "2", "4", "bogus"]:
            for pd in ["2", "3", "5"]:
                for wg in ["256", "512", "1024", "64"]:
                    monkeypatch.setenv("AQ_MATVEC_RC", rc)
                    monkeypatch.setenv("AQ_MATVEC_PD", pd)
                    monkeypatch.setenv("AQ_MATVEC_WG", wg)
                    err = normalized_error(qm.matvec(x), anchor, norms, x)
                    assert err < FP32_TOL, (rc, pd, wg, wpc, err)
        err = normalized_error(qm.matvec(x, kernel="fp32"), anchor, norms, x)
        assert err < FP32_TOL, ("fp32", wpc, err)


@pytest.mark.parametrize("dtype,shapes", [
    ("Q4_K", [(4096, 4096), (1024, 4096), (1024, 4096)]),     # fused q/k/v
    ("Q4_K", [(14336, 4096), (14336, 4096)]),                 # fused gate/up
    ("Q6_K", [(3, 2048), (7, 2048), (1, 2048), (500, 2048)]),  # ragged segments
    ("Q8_0", [(100, 4096)] * 8),
    ("Q5_K", [(64, 8192), (65, 8192)]),                       # two-step rows
    ("Q4_K", [(0, 4096), (300, 4096), (0, 4096), (5, 4096), (0, 4096)]),  # empty ones
])
def test_matvec_multi(dtype, shapes):
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_multi_device
    cols = shapes[0][1]
    x = synth.random_x(cols, seed=40)
    mats, datas = [], []
    for i, (r, c) in enumerate(shapes):
        datas.append(synth.random_matrix_bytes(dtype, r, c, seed=50 + i))
        mats.append(QuantMatrix(datas[-1], dtype, r, c))
    xd = torch.from_numpy(x).cuda()
    ys = [torch.full((r,), float("nan"), device="cuda") for r, _ in shapes]
    matvec_multi_device(mats, xd.data_ptr(), [y.data_ptr() for y in ys],
                        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    for qm, y, data, (r, c) in zip(mats, ys, datas, shapes):
        got = y.cpu().numpy()
        assert np.array_equal(got, qm.matvec(x))  # same kernel, same bits
        anchor, norms = _chunked_f64(data, dtype, r, c, x)
        assert normalized_error(got, anchor, norms, x) < FP32_TOL


def test_matvec_multi_rejects_mismatch():
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_multi_device
    a = QuantMatrix(synth.random_matrix_bytes("Q4_K", 8, 256, 1), "Q4_K", 8, 256)
    b = QuantMatrix(synth.random_matrix_bytes("Q8_0", 8, 256, 2), "Q8_0", 8, 256)
    c = QuantMatrix(synth.random_matrix_bytes("Q4_K", 8, 512, 3), "Q4_K", 8, 512)
    d = QuantMatrix(synth.random_matrix_bytes("Q4_K", 8, 256, 4), "Q4_K", 8, 256,
                    layout="split")
    xd = torch.zeros(512, device="cuda")
    y = torch.zeros(8, device="cuda")
    for pair in ([a, b], [a, c], [a, d]):
        with pytest.raises(ValueError):
            matvec_multi_device(pair, xd.data_ptr(), [y.data_ptr()] * 2)
    with pytest.raises(ValueError):
        matvec_multi_device([a] * 9, xd.data_ptr(), [y.data_ptr()] * 9)


# ------------------------------------------------------- row-pair mode ---

PAIR_CASES = [("Q4_K", 1, 2048), ("Q4_K", 3, 2048), ("Q4_K", 1001, 2048),
              ("Q6_K", 7, 2048), ("Q6_K", 2048, 1024), ("Q5_K", 999, 512),
              ("Q8_0", 513, 1024), ("Q4_0", 33, 32), ("Q5_1", 77, 640),
              ("Q4_K", 12345, 256)]


@pytest.mark.parametrize("dtype,rows,cols", PAIR_CASES)
def test_matvec_row_pairs(dtype, rows, cols, monkeypatch):
    """Rows of at most 32 lane units run two to a wave; the per-row sums
    (and so the results) are the same bits as one row per wave, and within
    tolerance of the oracle for odd row counts and every layout."""
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=rows + cols)
    x = synth.random_x(cols, seed=33)
    ref = RefMatrix(data, dtype, rows, cols)
    for layout in LAYOUTS.get(dtype, ["split"]):
        qm = QuantMatrix(data, dtype, rows, cols, layout=layout)
        monkeypatch.setenv("AQ_MATVEC_PAIR", "1")
        got = qm.matvec(x)
        monkeypatch.setenv("AQ_MATVEC_PAIR", "0")
        assert np.array_equal(got, qm.matvec(x))
        assert normalized_error(got, ref.matvec_f64(x), ref.row_norms(), x) < FP32_TOL


def test_matvec_row_pairs_multi_and_fused():
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_fused_device, matvec_multi_device
    shapes = [(3, 2048), (0, 2048), (2048, 2048), (511, 2048), (1, 2048)]
    x = synth.random_x(2048, seed=41)
    nw = np.random.default_rng(3).uniform(0.5, 1.5, 2048).astype(np.float32)
    mats = [QuantMatrix(synth.random_matrix_bytes("Q4_K", r, c, seed=60 + i), "Q4_K", r, c)
            for i, (r, c) in enumerate(shapes)]
    xd, nwd = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    ys = [torch.full((r,), float("nan"), device="cuda") for r, _ in shapes]
    s = torch.cuda.current_stream().cuda_stream
    matvec_multi_device(mats, xd.data_ptr(), [y.data_ptr() for y in ys], s)
    torch.cuda.synchronize()
    for qm, y in zip(mats, ys):
        assert np.array_equal(y.cpu().numpy(), qm.matvec(x))
    # residual accumulate into a base, RMSNorm prologue
    base = [torch.randn(r, device="cuda") for r, _ in shapes]
    ys = [b.clone() for b in base]
    matvec_fused_device(mats, xd.data_ptr(), [y.data_ptr() for y in ys], s,
                        norm_w_ptr=nwd.data_ptr(), eps=1e-5, rmsnorm=True, accumulate=True)
    torch.cuda.synchronize()
    xe = (x * np.float32(1.0 / np.sqrt(float(x.astype(np.float64) @ x) / 2048 + 1e-5))) * nw
    for qm, y, b, (r, c), i in zip(mats, ys, base, shapes, range(5)):
        ref = RefMatrix(synth.random_matrix_bytes("Q4_K", r, c, seed=60 + i), "Q4_K", r, c)
        want = ref.matvec_f64(xe) + b.cpu().numpy().astype(np.float64)
        assert normalized_error(y.cpu().numpy(), want, ref.row_norms(), xe) < FP32_TOL


@pytest.mark.parametrize("dtype,M,rows,cols", [("Q4_K", 300, 700, 4096), ("Q6_K", 64, 256, 2048),
                                               ("Q8_0", 129, 333, 1024), ("Q5_0", 70, 100, 4096)])
@pytest.mark.parametrize("splits", ["2", "3", "7"])
def test_matmul_t_split_k(dtype, M, rows, cols, splits, monkeypatch):
    """Contraction split over workgroups (partials summed in order): within
    the bf16 bar, and the same answer as without the split to fp32 rounding
    of the partial sums."""
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=M)
    X = synth.random_x(cols, seed=9, batch=M)
    qm = QuantMatrix(data, dtype, rows, cols)
    monkeypatch.setenv("AQ_MATMUL_SPLIT", "1")
    Y1 = qm.matmul_t(X, precision="bf16")
    monkeypatch.setenv("AQ_MATMUL_SPLIT", splits)
    Ys = qm.matmul_t(X, precision="bf16")
    W = qm.rows_at(np.arange(rows)).astype(np.float64)
    ref = X.astype(np.float64) @ W.T
    norms = np.linalg.norm(W, axis=1)
    assert normalized_error(Ys, ref, norms, X) < BF16_TOL
    assert normalized_error(Ys, Y1, norms, X) < 1e-5


@pytest.mark.parametrize("cols", [2048, 4096, 8192, 256])
@pytest.mark.parametrize("dtypes", [("Q4_K", "Q6_K"), ("Q5_K", "Q6_K"), ("Q4_K", "Q5_K")])
def test_matvec_mixed_formats(cols, dtypes):
    """Two dtypes in one launch (q/k and v of a Q4_K_M layer): every output is
    the same bits as the matrix's own matvec, for row pairs (K <= 2048),
    single-step and multi-step rows, ragged and empty segments, and with the
    RMSNorm prologue and the residual accumulation."""
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_fused_device, matvec_multi_device
    shapes = [(dtypes[0], 2048), (dtypes[0], 511), (dtypes[1], 512), (dtypes[1], 0), (dtypes[1], 3)]
    x = synth.random_x(cols, seed=cols)
    nw = np.random.default_rng(4).uniform(0.5, 1.5, cols).astype(np.float32)
    mats = [QuantMatrix(synth.random_matrix_bytes(d, r, cols, seed=70 + i), d, r, cols)
            for i, (d, r) in enumerate(shapes)]
    xd, nwd = torch.from_numpy(x).cuda(), torch.from_numpy(nw).cuda()
    s = torch.cuda.current_stream().cuda_stream
    ys = [torch.full((m.rows,), float("nan"), device="cuda") for m in mats]
    matvec_multi_device(mats, xd.data_ptr(), [y.data_ptr() for y in ys], s)
    torch.cuda.synchronize()
    for m, y in zip(mats, ys):
        assert np.array_equal(y.cpu().numpy(), m.matvec(x)), m.dtype
    base = [torch.randn(m.rows, device="cuda") for m in mats]
    ya = [b.clone() for b in base]
    matvec_fused_device(mats, xd.data_ptr(), [y.data_ptr() for y in ya], s,
                        norm_w_ptr=nwd.data_ptr(), eps=1e-5, rmsnorm=True, accumulate=True)
    yb = [b.clone() for b in base]
    for m, y in zip(mats, yb):  # one launch per matrix, same prologue
        matvec_fused_device([m], xd.data_ptr(), [y.data_ptr()], s, norm_w_ptr=nwd.data_ptr(),
                            eps=1e-5, rmsnorm=True, accumulate=True)
    torch.cuda.synchronize()
    for a, b in zip(ya, yb):
        assert torch.equal(a, b)


@pytest.mark.parametrize("cols", [2048, 4096, 8192])
def test_matvec_launch_rows_do_not_change_bits(cols):
    """The launch shape follows the launch's row count (workgroup size, rows in
    flight), and a launch of 4,615 rows crosses every such threshold against
    launches of 4,096, 512 and 7 rows: plain, RMSNorm-staged and SwiGLU-staged
    products must still be the bits of one launch per matrix."""
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_fused_device
    rows = [4096, 512, 7]
    x = synth.random_x(cols, seed=cols + 1)
    x2 = synth.random_x(cols, seed=cols + 2)
    nw = np.random.default_rng(5).uniform(0.5, 1.5, cols).astype(np.float32)
    mats = [QuantMatrix(synth.random_matrix_bytes("Q4_K", r, cols, seed=90 + i), "Q4_K", r, cols)
            for i, r in enumerate(rows)]
    xd, x2d, nwd = (torch.from_numpy(a).cuda() for a in (x, x2, nw))
    s = torch.cuda.current_stream().cuda_stream
    for mode in ({}, {"rmsnorm": True}, {"swiglu": True}):
        print(f"launch rows {rows} cols={cols} {mode}", flush=True)
        kw = dict(x2_ptr=x2d.data_ptr(), norm_w_ptr=nwd.data_ptr(), eps=1e-5, **mode)
        ya = [torch.full((r,), float("nan"), device="cuda") for r in rows]
        matvec_fused_device(mats, xd.data_ptr(), [y.data_ptr() for y in ya], s, **kw)
        yb = [torch.full((r,), float("nan"), device="cuda") for r in rows]
        for m, y in zip(mats, yb):
            matvec_fused_device([m], xd.data_ptr(), [y.data_ptr()], s, **kw)
        torch.cuda.synchronize()
        for a, b in zip(ya, yb):
            assert torch.equal(a, b), mode


def test_matvec_mixed_rejects_unsupported():
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_fused_device, matvec_multi_device
    a = QuantMatrix(synth.random_matrix_bytes("Q4_K", 8, 256, 1), "Q4_K", 8, 256)
    b = QuantMatrix(synth.random_matrix_bytes("Q6_K", 8, 256, 2), "Q6_K", 8, 256)
    xd = torch.zeros(256, device="cuda")
    y = torch.zeros(8, device="cuda")
    for mats in ([b, a], [a, b, a]):  # order: first dtype first, one switch
        with pytest.raises(ValueError):
            matvec_multi_device(mats, xd.data_ptr(), [y.data_ptr()] * len(mats))
    with pytest.raises(ValueError, match="SwiGLU"):
        matvec_fused_device([a, b], xd.data_ptr(), [y.data_ptr()] * 2, x2_ptr=xd.data_ptr(),
                            swiglu=True)


@pytest.mark.parametrize("M,rows,cols", [(512, 4096, 4096), (64, 300, 1024), (130, 65, 96),
                                         (1, 17, 32), (200, 128, 8192)])
def test_matmul_t_int8_q8_0(M, rows, cols):
    """Q8_0 against int8 activations: within 1e-5 of the scheme computed in
    float64 (exact integer block dots, fp32 scaling), and within the 1e-2
    prefill bar of the true product."""
    print(f"int8 matmul_t Q8_0 M={M} {rows}x{cols}", flush=True)
    data = synth.random_matrix_bytes("Q8_0", rows, cols, seed=M + cols)
    X = synth.random_x(cols, seed=11, batch=M)
    X[0, :32] = 0.0  # an all-zero block
    qm = QuantMatrix(data, "Q8_0", rows, cols)
    Y = qm.matmul_t(X, precision="int8")
    ref = RefMatrix(data, "Q8_0", rows, cols)
    norms = ref.row_norms()
    assert normalized_error(Y, ref.matmul_t_int8_f64(X), norms, X) < 1e-5
    assert normalized_error(Y, ref.matmul_t_f64(X), norms, X) < BF16_TOL


def test_matmul_t_int8_needs_q8_0():
    qm = QuantMatrix(synth.random_matrix_bytes("Q4_K", 4, 256, 0), "Q4_K", 4, 256)
    with pytest.raises(ValueError, match="Q8_0"):
        qm.matmul_t(np.zeros((2, 256), np.float32), precision="int8")


# ------------------------------------------------------- edge shapes ---

@pytest.mark.parametrize("dtype", ["Q4_K", "Q8_0", "F16"])
def test_empty_matrices(dtype):
    """Zero rows or zero columns: empty outputs, zeros for W x with K = 0
    (the reference's empty-matrix behaviour), IndexError for any row."""
    from alpacca_amd.qmatrix import DENSE_DTYPES, DenseMatrix
    make = (lambda r, c: DenseMatrix(b"", dtype, r, c)) if dtype in DENSE_DTYPES else \
        (lambda r, c: QuantMatrix(b"", dtype, r, c))
    W = make(0, 256)
    assert W.matvec(np.ones(256, np.float32)).shape == (0,)
    assert W.matmul_t(np.ones((3, 256), np.float32)).shape == (3, 0)
    assert W.rows_at([]).shape == (0, 256)
    with pytest.raises(IndexError):
        W.row(0)
    W0 = make(5, 0)
    assert np.array_equal(W0.matvec(np.zeros(0, np.float32)), np.zeros(5, np.float32))
    assert np.array_equal(W0.matmul_t(np.zeros((2, 0), np.float32)), np.zeros((2, 5), np.float32))
    assert W0.rows_at([4, 0]).shape == (2, 0)


@pytest.mark.parametrize("kernel", ["int8", "fp32"])
@pytest.mark.parametrize("dtype", ["Q4_K", "Q6_K", "Q8_0"])
@pytest.mark.parametrize("cols", [53248, 65536])
def test_matvec_wide_rows(dtype, cols, kernel):
    """Every K that can_quantized_matvec accepts runs (qmatrix.py:148-171,
    :350-352 put no upper bound on K).  Both kernels stage x in LDS, so a
    row wider than one launch can stage is cut into column windows whose
    products are added in K order; the result stays within the fp32 bar of
    the float64 product (K = 53,248 is a 405B-class ffn_down)."""
    rows = 40
    data = synth.random_matrix_bytes(dtype, rows, cols, seed=cols % 997)
    W, ref = QuantMatrix(data, dtype, rows, cols), RefMatrix(data, dtype, rows, cols)
    x = synth.random_x(cols, seed=cols % 991)
    y = W.matvec(x, kernel=kernel)
    assert normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x) < FP32_TOL
    # windows are disjoint: x zero outside one block picks out that block's column range
    be = Q.GEOMETRY[dtype][0]
    xb = np.zeros(cols, np.float32)
    xb[-be:] = x[-be:]
    yb = W.matvec(xb, kernel=kernel)
    assert normalized_error(yb, ref.matvec_f64(xb), ref.row_norms(), xb) < FP32_TOL


def test_matvec_wide_rows_multi_and_fused():
    """The one-launch forms take wide rows too: several matrices sharing x,
    the residual accumulate and the SwiGLU-staged input each window by
    window; an RMSNorm-staged input needs all of x in one launch and is
    refused with ValueError."""
    torch = pytest.importorskip("torch")
    from alpacca_amd.qmatrix import matvec_fused_device, matvec_multi_device
    K = 53248
    shapes = [(24, K), (9, K)]
    datas = [synth.random_matrix_bytes("Q4_K", r, c, seed=70 + i) for i, (r, c) in enumerate(shapes)]
    mats = [QuantMatrix(d, "Q4_K", r, c) for d, (r, c) in zip(datas, shapes)]
    refs = [RefMatrix(d, "Q4_K", r, c) for d, (r, c) in zip(datas, shapes)]
    g, u = synth.random_x(K, seed=71), synth.random_x(K, seed=72)
    gd, ud = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    s = torch.cuda.current_stream().cuda_stream
    ys = [torch.full((r,), float("nan"), device="cuda") for r, _ in shapes]
    matvec_multi_device(mats, gd.data_ptr(), [y.data_ptr() for y in ys], s)
    torch.cuda.synchronize()
    for ref, y in zip(refs, ys):
        assert normalized_error(y.cpu().numpy(), ref.matvec_f64(g), ref.row_norms(), g) < FP32_TOL
    base = [torch.randn(r, device="cuda") for r, _ in shapes]
    ys = [b.clone() for b in base]
    matvec_fused_device(mats, gd.data_ptr(), [y.data_ptr() for y in ys], s,
                        x2_ptr=ud.data_ptr(), swiglu=True, accumulate=True)
    torch.cuda.synchronize()
    with np.errstate(over="ignore"):
        xe = (g / (np.float32(1.0) + np.exp(-g)) * u).astype(np.float32)
    for ref, y, b in zip(refs, ys, base):
        want = ref.matvec_f64(xe) + b.cpu().numpy().astype(np.float64)
        assert normalized_error(y.cpu().numpy(), want, ref.row_norms(), xe) < FP32_TOL
    nwd = torch.ones(K, device="cuda")
    with pytest.raises(ValueError, match="RMSNorm-staged"):
        matvec_fused_device(mats, gd.data_ptr(), [y.data_ptr() for y in ys], s,
                            norm_w_ptr=nwd.data_ptr(), eps=1e-5, rmsnorm=True)
