"""Decode attention against a float64 softmax at long contexts and wide score
ranges.  The attention weights are e^(s - max) computed as
2^((s - max) log2 e) on the hardware exp2, whose rounded product adds a
relative error of about |s - max| 2^-24 ln 2 to each weight; this pins the
resulting error of the outputs where the scores span tens of units (the
reference computes float32 np.exp, model.py:447-455; the bar is taken
against float64, the exact softmax)."""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from alpacca_amd import _lib

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def _attention_f64(q, K, V, group):
    """q (n_head, hd), K/V (n_pos, n_kv, hd): the exact softmax attention."""
    n_head, hd = q.shape
    out = np.empty((n_head, hd))
    for h in range(n_head):
        kv = h // group
        s = K[:, kv, :].astype(np.float64) @ q[h].astype(np.float64) / np.sqrt(hd)
        w = np.exp(s - s.max())
        out[h] = (w @ V[:, kv, :].astype(np.float64)) / w.sum()
    return out


@pytest.mark.parametrize("n_ctx,pos,q_scale", [(2304, 2303, 1.0), (2304, 2175, 12.0),
                                               (4096, 4095, 25.0), (8192, 6000, 6.0)])
@pytest.mark.parametrize("hd", [64, 128])
def test_attention_vs_f64_wide_scores(n_ctx, pos, q_scale, hd):
    """Scores with standard deviations of about 1, 12, 25 and 6 units (q
    scaled; keys ~ N(0, 1)): outputs within 1e-5 of max|V| of the float64
    softmax, and the measured maximum printed for the record."""
    n_head, n_kv = 32, 8
    rng = np.random.default_rng(n_ctx + hd + int(q_scale))
    q = (rng.standard_normal((n_head, hd)) * q_scale).astype(np.float32)
    K = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    V = rng.standard_normal((n_ctx, n_kv, hd)).astype(np.float32)
    d = torch.device("cuda", 0)
    kc = torch.from_numpy(np.ascontiguousarray(K.transpose(1, 0, 2))).to(d)
    vc = torch.from_numpy(np.ascontiguousarray(V.transpose(1, 0, 2))).to(d)
    qd = torch.from_numpy(q.reshape(-1)).to(d)
    out = torch.empty(n_head * hd, device=d)
    P = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    lib = _lib.ensure_device()
    _lib.check(lib.aq_attention(P(qd), P(kc), P(vc), n_head, n_kv, hd, n_ctx, None, pos,
                                P(out), None))
    got = out.cpu().numpy().reshape(n_head, hd).astype(np.float64)
    want = _attention_f64(q, K[:pos + 1], V[:pos + 1], n_head // n_kv)
    err = np.abs(got - want).max() / np.abs(V).max()
    s_span = float(np.abs(q).max() * np.sqrt(hd))
    print(f"attention n_ctx={n_ctx} pos={pos} hd={hd} q_scale={q_scale}: "
          f"max|out - f64| / max|V| = {err:.2e}", flush=True)
    assert err < 1e-5, (err, s_span)
