"""The C-ABI boundary and the host mirror, without a GPU: the library loads,
exports every entry point include/alpacca_amd.h declares, validates arguments
with the reference's exception classes before touching a device, and the
product never falls back to the CPU (or to oracle/)."""
from __future__ import annotations

import ast
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from alpacca_amd import _lib
from alpacca_amd import synth
from alpacca_amd.quants import QUANT_GEOMETRY

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "alpacca_amd.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return set(re.findall(r"\b(aq_[a-z0-9_]+)\s*\(", text))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert {"aq_matrix_create", "aq_matvec", "aq_matmul_t", "aq_dequant_rows",
            "aq_matvec_multi", "aq_last_error"} <= names
    for name in names:
        assert hasattr(lib, name), name
    assert names == set(_lib.SIGNATURES), "ctypes signatures out of sync with the header"


def test_dtype_ids_match_header_and_ggml():
    text = HEADER.read_text()
    for name, ident in _lib.DTYPE_IDS.items():
        macro = "AQ_" + name
        m = re.search(rf"#define {macro} (\d+)", text)
        assert m and int(m.group(1)) == ident


def test_geometry_matches_reference_table():
    lib = _lib.load()
    for dtype, (be, bb, sub, aff) in QUANT_GEOMETRY.items():
        out = [ctypes.c_int() for _ in range(4)]
        assert lib.aq_geometry(_lib.DTYPE_IDS[dtype], *[ctypes.byref(o) for o in out]) == 0
        assert [o.value for o in out] == [be, bb, sub, int(aff)]
    assert lib.aq_geometry(99, None, None, None, None) == _lib.AQ_ERR_VALUE
    assert b"does not support" in lib.aq_last_error()


def test_create_validates_before_touching_a_device():
    lib = _lib.load()
    h = ctypes.c_void_p()
    buf = (ctypes.c_uint8 * 144)()
    assert lib.aq_matrix_create(buf, 144, 12, 1, 256, 0, None) == _lib.AQ_ERR_VALUE
    assert lib.aq_matrix_create(buf, 144, 99, 1, 256, 0, ctypes.byref(h)) == _lib.AQ_ERR_VALUE
    assert lib.aq_matrix_create(buf, 144, 12, 1, 255, 0, ctypes.byref(h)) == _lib.AQ_ERR_VALUE
    assert b"multiple of 256" in lib.aq_last_error()
    assert lib.aq_matrix_create(buf, 143, 12, 1, 256, 0, ctypes.byref(h)) == _lib.AQ_ERR_VALUE
    assert b"expected 144" in lib.aq_last_error()
    assert lib.aq_matrix_create(buf, 210, 14, 1, 256, 1, ctypes.byref(h)) == _lib.AQ_ERR_VALUE
    assert lib.aq_matrix_create(buf, 144, 12, -1, 256, 0, ctypes.byref(h)) == _lib.AQ_ERR_VALUE
    assert h.value is None


def test_host_mirror_raises_reference_errors():
    from alpacca_amd.qmatrix import QuantMatrix
    data = synth.random_matrix_bytes("Q4_K", 2, 256, 0)
    with pytest.raises(ValueError, match="does not support"):
        QuantMatrix(data, "Q3_K", 2, 256)
    with pytest.raises(ValueError, match="multiple of 256"):
        QuantMatrix(data, "Q4_K", 2, 200)
    with pytest.raises(ValueError, match="expected 288"):
        QuantMatrix(data[:-1], "Q4_K", 2, 256)


@pytest.mark.skipif(_lib.device_count() > 0, reason="a GPU is visible")
def test_no_cpu_fallback_without_gpu():
    from alpacca_amd.qmatrix import QuantMatrix
    data = synth.random_matrix_bytes("Q4_K", 2, 256, 0)
    with pytest.raises(RuntimeError, match="no HIP device"):
        QuantMatrix(data, "Q4_K", 2, 256)


def test_dispatch_seam_dense_path_and_module_surface():
    from alpacca_amd import qmatrix, tensor as T
    W = np.array([[1.0, -2.0, 0.5], [3.0, 4.0, -1.0]], dtype=np.float32)
    assert np.allclose(T.matvec(W, np.array([2.0, -1.0, 4.0], np.float32)), [6.0, -2.0])
    assert np.allclose(T.matmul_t(np.ones((2, 3)), W), [[-0.5, 6.0], [-0.5, 6.0]])
    assert np.array_equal(T.matrix_row(W, 1), W[1])
    assert np.array_equal(T.matrix_rows(W, [1, 0]), W[[1, 0]])
    assert T.can_quantized_matvec("Q4_K", 512) and not T.can_quantized_matvec("Q4_K", 500)
    assert not T.can_quantized_matvec("F16", 512)
    assert qmatrix.QUANTIZED_MATVEC_DTYPES == frozenset(QUANT_GEOMETRY)
    assert T.hot_cache_stats() == {"limit_bytes": 0, "used_bytes": 0, "matrices": 0}
    T._reset_hot_cache_state()
    assert qmatrix.QMatrix is qmatrix.QuantMatrix is T.QuantizedMatrix


def test_product_never_imports_the_oracle():
    for path in (ROOT / "alpacca_amd").rglob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            names = []
            if isinstance(node, ast.Import):
                names = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom):
                names = [node.module or ""]
            assert not any(n == "oracle" or n.startswith("oracle.") for n in names), path


def test_bench_refuses_several_gpus():
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "single GPU" in r.stderr


def test_interleave_rows_and_pair_support():
    """Host helpers of the SwiGLU-pairs gate/up launch: the interleaved
    matrix decodes to gate row i at 2i and up row i at 2i+1 (checked through
    the oracle's decoder), and pair_rows_supported follows the integer
    kernel's two-rows-per-wave limit (32 lane units: K <= 2048 for the
    K-quants, <= 1024 for the 32-element formats)."""
    import numpy as np

    from alpacca_amd import synth
    from alpacca_amd.qmatrix import interleave_rows, pair_rows_supported
    from oracle.qmatrix_ref import RefMatrix
    for dtype, cols in (("Q4_K", 512), ("Q6_K", 256), ("Q8_0", 96), ("Q5_1", 64)):
        a = synth.random_matrix_bytes(dtype, 5, cols, seed=1)
        b = synth.random_matrix_bytes(dtype, 5, cols, seed=2)
        gu = interleave_rows(a, b, 5, cols, dtype)
        assert gu.dtype == np.uint8 and gu.size == 2 * len(a)
        dense = RefMatrix(gu.tobytes(), dtype, 10, cols).dense()
        assert np.array_equal(dense[0::2], RefMatrix(a, dtype, 5, cols).dense())
        assert np.array_equal(dense[1::2], RefMatrix(b, dtype, 5, cols).dense())
    assert pair_rows_supported("Q4_K", 2048) and not pair_rows_supported("Q4_K", 4096)
    assert pair_rows_supported("Q6_K", 2048) and not pair_rows_supported("Q5_K", 2304)
    assert pair_rows_supported("Q8_0", 1024) and not pair_rows_supported("Q8_0", 1056)
    assert not pair_rows_supported("Q4_K", 300)  # not a whole number of blocks
    assert not pair_rows_supported("F32", 256)   # dense: the fp32 kernel has no pairs


def _ctx_lengths():
    """Cache lengths 1 .. 131,072: every length up to 300, then each power of
    two with its neighbours, the chunk and split boundaries they cross."""
    out = set(range(1, 301))
    p = 256
    while p <= 131072:
        out.update({p - 1, p, p + 1, p + 31, p + 63})
        p *= 2
    out.update({2047, 2048, 2049, 2304, 8191, 8192, 131071, 131072})
    return sorted(n for n in out if 1 <= n <= 131072)


def test_attention_scratch_covers_every_launch_form():
    """The partial scratch the library sizes for a decode-attention call equals
    the extent the call's launch grid writes (split kernel for one query token,
    chunked kernel for several), for every supported head_dim and group and
    cache lengths 1 .. 131,072; the launchers refuse a smaller scratch."""
    lib = _lib.load()
    sb, lb = ctypes.c_size_t(), ctypes.c_size_t()
    checked = 0
    for hd in (64, 128):
        ch = 64 if hd == 64 else 32          # positions per chunk
        for n_kv, group in ((1, 1), (8, 1), (8, 4), (4, 8), (2, 2)):
            for T in (1, 2, 17):
                for n_ctx in _ctx_lengths():
                    rc = lib.aq_attention_scratch_info(n_kv * group, n_kv, hd, n_ctx, T,
                                                       ctypes.byref(sb), ctypes.byref(lb))
                    assert rc == _lib.AQ_OK, lib.aq_last_error()
                    assert sb.value == lb.value, (hd, n_kv, group, T, n_ctx)
                    # closed form: one partial (hd + 4 floats) per query head and
                    # split (T = 1: min(32, max(1, chunks // 2))) or per chunk and token
                    chunks = -(-n_ctx // ch)
                    slots = min(32, max(1, chunks // 2)) if T == 1 else chunks
                    assert lb.value == T * n_kv * group * slots * (hd + 4) * 4
                    checked += 1
    assert checked > 10000
    assert lib.aq_attention_scratch_info(32, 8, 96, 100, 1, None, None) == _lib.AQ_ERR_VALUE
    assert lib.aq_attention_scratch_info(32, 8, 64, 0, 1, None, None) == _lib.AQ_ERR_VALUE
