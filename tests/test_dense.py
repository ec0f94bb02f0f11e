"""Dense F32 / F16 / BF16 matrices (DenseMatrix): the reference keeps such
weights as float32 arrays and multiplies with NumPy (model.py:269-281,
quants.py:517-523, tensor.py:82-113).

The oracle's decode is pinned by known bit patterns (IEEE half and bfloat16
encodings of exact values, subnormals, signed zero, infinity); the device
path by the f64 product over the same decoded values (2e-5 / 1e-2
normalized), exact row gathers, and greedy tokens of a
model with dense matrices equal to the oracle's.
"""
from __future__ import annotations

import numpy as np
import pytest

from alpacca_amd import gguf, synth
from alpacca_amd.qmatrix import DENSE_DTYPES, DenseMatrix, QuantMatrix
from oracle.qmatrix_ref import DenseRef, normalized_error
from oracle.quants_ref import dense_decode

DENSE = ("F32", "F16", "BF16")


def test_dense_decode_known_answers():
    f16 = np.array([0x3C00, 0xC000, 0x0001, 0x7BFF, 0x8000, 0x7C00, 0x3555], "<u2")
    got = dense_decode(f16.view(np.uint8).tobytes(), f16.size, "F16")
    want = [1.0, -2.0, 2.0 ** -24, 65504.0, -0.0, np.inf, 1365 / 4096]
    assert np.array_equal(got, np.array(want, np.float32))
    assert np.signbit(got[4])
    bf = np.array([0x3F80, 0xC040, 0x0001, 0x7F7F, 0x3EAB], "<u2")
    got = dense_decode(bf.view(np.uint8).tobytes(), bf.size, "BF16")
    want = np.array([0x3F800000, 0xC0400000, 0x00010000, 0x7F7F0000, 0x3EAB0000],
                    np.uint32).view(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0] == 1.0 and got[1] == -3.0
    f32 = np.array([1.5, -0.0, 3.4e38, 1e-45], np.float32)
    assert np.array_equal(dense_decode(f32.tobytes(), 4, "F32").view(np.uint32), f32.view(np.uint32))
    with pytest.raises(ValueError):
        dense_decode(b"\0" * 6, 4, "F16")


def test_synth_bf16_rounds_to_nearest_even():
    v = synth.dense_values_bytes("BF16", 4, 64, seed=3).view("<u2")
    ref = np.random.default_rng(3).standard_normal(256).astype(np.float32) * np.float32(0.02)
    back = (v.astype(np.uint32) << 16).view(np.float32)
    # |error| at most half a bf16 ulp (2^-8 relative)
    assert np.all(np.abs(back - ref) <= np.abs(ref) * 2.0 ** -8)


@pytest.mark.parametrize("dtype", DENSE)
def test_dense_matrix_rejects_bad_arguments(dtype):
    w = DENSE_DTYPES[dtype]
    with pytest.raises(ValueError, match="multiple of 32"):
        DenseMatrix(b"\0" * (4 * 48 * w), dtype, 4, 48)
    with pytest.raises(ValueError, match="bytes, expected"):
        DenseMatrix(b"\0" * (4 * 64 * w - 2), dtype, 4, 64)
    with pytest.raises(ValueError, match="not Q4_K"):
        DenseMatrix(b"\0" * 64, "Q4_K", 1, 32)
    with pytest.raises(ValueError):  # QuantMatrix keeps the reference's rejection
        QuantMatrix(b"\0" * (4 * 64 * w), dtype, 4, 64)


def test_gguf_keeps_dense_matrices(tmp_path):
    from alpacca_amd.model import Tensor, synthetic_llama_1b
    hp, tensors = synthetic_llama_1b(seed=1, n_layer=1, n_embd=256, n_head=2, n_kv=1,
                                     n_ff=512, n_vocab=96, n_ctx_train=256)
    tensors["blk.0.attn_q.weight"] = Tensor("F16", (256, 256), synth.dense_values_bytes("F16", 256, 256, 1))
    tensors["blk.0.ffn_up.weight"] = Tensor("BF16", (512, 256), synth.dense_values_bytes("BF16", 512, 256, 2))
    f32 = np.random.default_rng(4).standard_normal((96, 256)).astype(np.float32)
    tensors["output.weight"] = Tensor("F32", (96, 256), f32)
    p = tmp_path / "d.gguf"
    gguf.write_model(p, hp, tensors)
    with gguf.GGUFReader(p) as g:
        assert g.tensors["blk.0.attn_q.weight"].dtype == "F16"
        back = gguf.read_tensors(g)
        assert back["blk.0.attn_q.weight"].dtype == "F16"
        assert bytes(back["blk.0.attn_q.weight"].data) == tensors["blk.0.attn_q.weight"].data.tobytes()
        assert bytes(back["blk.0.ffn_up.weight"].data) == tensors["blk.0.ffn_up.weight"].data.tobytes()
        assert back["output.weight"].dtype == "F32" and back["output.weight"].shape == (96, 256)
        assert bytes(back["output.weight"].data) == f32.tobytes()
        assert back["blk.0.attn_norm.weight"].data.dtype == np.float32
        del back


# ---------------------------------------------------------------- GPU parity --

SHAPES = [(64, 32), (300, 512), (2048, 2048), (4096, 4096), (96, 14336)]


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DENSE)
@pytest.mark.parametrize("rows,cols", SHAPES)
def test_dense_matvec_vs_f64(dtype, rows, cols):
    data = synth.dense_values_bytes(dtype, rows, cols, seed=rows + cols, std=1.0)
    W = DenseMatrix(data, dtype, rows, cols)
    ref = DenseRef(data, dtype, rows, cols)
    x = synth.random_x(cols, seed=cols)
    y = W.matvec(x)
    assert normalized_error(y, ref.matvec_f64(x), ref.row_norms(), x) < 2e-5
    assert np.array_equal(W.rows_at([0, rows - 1, rows // 2]), ref.rows_at([0, rows - 1, rows // 2]))
    with pytest.raises(IndexError):
        W.row(rows)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", DENSE)
@pytest.mark.parametrize("M", [5, 70, 512])
def test_dense_matmul_t_vs_f64(dtype, M):
    rows, cols = 1000, 2048
    data = synth.dense_values_bytes(dtype, rows, cols, seed=M, std=1.0)
    W = DenseMatrix(data, dtype, rows, cols)
    ref = DenseRef(data, dtype, rows, cols)
    X = synth.random_x(cols, seed=M, batch=M)
    want = ref.matmul_t_f64(X)
    norms = ref.row_norms()
    for prec, tol in (("fp32", 2e-5), ("bf16", 1e-2)):
        Y = W.matmul_t(X, precision=prec)
        err = max(normalized_error(Y[i], want[i], norms, X[i]) for i in range(M))
        assert err < tol, (prec, err)


@pytest.mark.gpu
def test_dense_rejected_by_multi_launches():
    import torch
    from alpacca_amd.qmatrix import matvec_multi_device
    W = DenseMatrix(synth.dense_values_bytes("F16", 64, 64), "F16", 64, 64)
    x = torch.zeros(64, device="cuda")
    y = torch.zeros(64, device="cuda")
    with pytest.raises(ValueError, match="aq_matvec"):
        matvec_multi_device([W], x.data_ptr(), [y.data_ptr()])


@pytest.mark.gpu
@pytest.mark.parametrize("dense", ["F16", "BF16", "F32"])
def test_model_with_dense_matrices_greedy(tmp_path, dense):
    """Some matrices dense (the reference's F16 / F32 GGUFs), the rest
    quantized: greedy tokens equal the oracle's, also through a GGUF file."""
    from alpacca_amd.model import Model, Tensor, synthetic_llama_1b
    from oracle.model_ref import RefModel
    hp, tensors = synthetic_llama_1b(seed=7, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=700, n_ctx_train=512)
    for i, name in enumerate(["blk.0.attn_q.weight", "blk.0.ffn_down.weight",
                              "blk.1.attn_v.weight", "blk.1.ffn_gate.weight",
                              "token_embd.weight"]):
        rows, cols = tensors[name].shape
        tensors[name] = Tensor(dense, (rows, cols),
                               synth.dense_values_bytes(dense, rows, cols, seed=50 + i))
    prompt = list(np.random.default_rng(11).integers(0, hp.n_vocab, 40))
    m = Model(hp, tensors)
    assert not m.fused
    toks = m.generate_greedy(prompt, 12)
    ref_toks, margins = RefModel(hp, tensors).greedy(prompt, 12)
    assert toks == ref_toks, (toks, ref_toks, min(margins))
    p = tmp_path / "m.gguf"
    gguf.write_model(p, hp, tensors)
    assert gguf.load_model(p).generate_greedy(prompt, 12) == toks
