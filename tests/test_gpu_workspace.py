"""The library's per-stream scratch (workspace) across HIP graph capture:
a call that needs scratch, run once eagerly, can then be captured; the
captured buffer outlives aq_release_workspace and a larger eager call, so
the graph keeps replaying the same bits; and a call that would need more
scratch than the stream holds is refused while the stream is capturing
(nothing is allocated under capture), with a message that says what to do."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from alpacca_amd import _lib, synth
from alpacca_amd.qmatrix import QuantMatrix

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def test_captured_scratch_survives_release_and_growth():
    d = torch.device("cuda", 0)
    rows, cols, M = 2048, 2048, 16  # the exact-fp16 kernel: X pieces and split partials
    qm = QuantMatrix(synth.random_matrix_bytes("Q4_K", rows, cols, seed=1), "Q4_K", rows, cols)
    X = torch.from_numpy(synth.random_x(cols, seed=2, batch=M)).to(d)
    Y = torch.empty((M, rows), device=d)
    s = torch.cuda.Stream(d)
    h = s.cuda_stream
    lib = _lib.ensure_device()
    lib.aq_release_workspace(ctypes.c_void_p(h))  # start from no scratch on this stream
    with torch.cuda.stream(s):
        qm.matmul_t_device(X.data_ptr(), M, Y.data_ptr(), h)  # eager: sizes the scratch
    s.synchronize()
    want = Y.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        qm.matmul_t_device(X.data_ptr(), M, Y.data_ptr(), h)
    for _ in range(3):
        Y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(Y, want)
    # release, then a larger eager call on the same stream (new, larger scratch)
    _lib.check(lib.aq_release_workspace(ctypes.c_void_p(h)))
    X2 = torch.from_numpy(synth.random_x(cols, seed=3, batch=8 * M)).to(d)
    Y2 = torch.empty((8 * M, rows), device=d)
    with torch.cuda.stream(s):
        qm.matmul_t_device(X2.data_ptr(), 8 * M, Y2.data_ptr(), h)
    s.synchronize()
    for _ in range(3):
        Y.zero_()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        assert torch.equal(Y, want)
    # the stream works eagerly as before
    with torch.cuda.stream(s):
        qm.matmul_t_device(X.data_ptr(), M, Y.data_ptr(), h)
    s.synchronize()
    assert torch.equal(Y, want)


def test_capture_refuses_scratch_growth():
    """Under capture the call fails on the host (no kernel is launched) and
    names the remedy; the stream is usable afterwards."""
    d = torch.device("cuda", 0)
    rows, cols = 2048, 2048
    qm = QuantMatrix(synth.random_matrix_bytes("Q4_K", rows, cols, seed=4), "Q4_K", rows, cols)
    s = torch.cuda.Stream(d)
    h = s.cuda_stream
    lib = _lib.ensure_device()
    lib.aq_release_workspace(ctypes.c_void_p(h))
    X = torch.from_numpy(synth.random_x(cols, seed=5, batch=64)).to(d)
    Y = torch.empty((64, rows), device=d)
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError, match="eagerly before capture"):
        with torch.cuda.graph(g, stream=s):
            qm.matmul_t_device(X.data_ptr(), 64, Y.data_ptr(), h)
    with torch.cuda.stream(s):
        qm.matmul_t_device(X.data_ptr(), 64, Y.data_ptr(), h)
    s.synchronize()
    ref = qm.matmul_t(X.cpu().numpy())
    assert np.array_equal(Y.cpu().numpy(), ref)
