"""Pins the decode-step oracle (oracle/model_ref.py) on the CPU.

Each restated function is checked against something other than itself:
closed forms (rotation of unit vectors, RMS of the output, softmax of one
key), brute-force loops, the independent pure-Python decoder
(model.py:557-608), the reference's own differential bar for batched vs
sequential decoding (< 1e-4, tests/smoke.py:950-972), and planted mistakes
that those checks must catch.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

from alpacca_amd import synth
from alpacca_amd.model import Hyperparams, synthetic_llama_1b
from oracle import model_ref as MR
from oracle import quants_ref as Q


def _hp(style="norm", n_rot=8, hd=8, n_head=4, n_kv=2, base=10000.0):
    return Hyperparams(arch="llama", n_layer=1, n_embd=n_head * hd, n_head=n_head,
                       n_kv=n_kv, n_ff=64, n_vocab=32, n_ctx_train=64, head_dim=hd,
                       n_rot=n_rot, rms_eps=1e-5, rope_base=base, rope_style=style)


@pytest.fixture(scope="module")
def tiny():
    hp, tensors = synthetic_llama_1b(seed=3, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=512, n_ctx_train=128)
    return hp, tensors


def test_rope_tables_closed_form():
    hp = _hp(base=500000.0, n_rot=64, hd=64)
    cos, sin = MR.rope_tables(hp, 100)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)  # angle 0
    assert np.allclose(cos ** 2 + sin ** 2, 1.0, atol=1e-6)
    # pair 0 rotates by exactly pos radians (inv_freq[0] = 1)
    assert np.allclose(cos[:, 0], np.cos(np.arange(100)), atol=1e-6)
    # inv_freq[i] = base^(-2i/n_rot)
    i = 7
    assert np.isclose(np.arctan2(sin[1, i], cos[1, i]), 500000.0 ** (-2 * i / 64), rtol=1e-5)


@pytest.mark.parametrize("style", ["norm", "neox"])
def test_rope_rotates_unit_vectors(style):
    hp = _hp(style=style)
    cos, sin = MR.rope_tables(hp, 16)
    half = hp.n_rot // 2
    for i in range(half):
        a, b = (2 * i, 2 * i + 1) if style == "norm" else (i, i + half)
        e = np.zeros(hp.n_head * hp.head_dim, np.float32)
        e[a] = 1.0  # (1, 0) of pair i in head 0 -> (cos, sin)
        out = MR.rope_np(e, hp.n_head, 5, hp, cos, sin)
        assert out[a] == cos[5, i] and out[b] == sin[5, i]
        assert np.count_nonzero(out) <= 2


def test_rope_keeps_norms_and_untouched_tail():
    hp = _hp(n_rot=4, hd=8)
    cos, sin = MR.rope_tables(hp, 16)
    v = np.random.default_rng(0).standard_normal(hp.n_head * hp.head_dim).astype(np.float32)
    out = MR.rope_np(v, hp.n_head, 9, hp, cos, sin).reshape(hp.n_head, hp.head_dim)
    vin = v.reshape(hp.n_head, hp.head_dim)
    assert np.array_equal(out[:, 4:], vin[:, 4:])  # dims past n_rot
    for i in range(2):
        assert np.allclose(np.hypot(out[:, 2 * i], out[:, 2 * i + 1]),
                           np.hypot(vin[:, 2 * i], vin[:, 2 * i + 1]), rtol=1e-6)
    # the batched form at positions (9, 9) equals the single form
    pb = MR.rope_batch_np(np.stack([v, v]), hp.n_head, np.array([9, 9]), hp, cos, sin)
    assert np.array_equal(pb[0], out.reshape(-1))


def test_rmsnorm_known_answers():
    x = np.array([3.0, 4.0], np.float32)
    w = np.array([1.0, 2.0], np.float32)
    inv = 1.0 / math.sqrt(12.5 + 1e-5)
    assert np.allclose(MR.rmsnorm(x, w, 1e-5), [3 * inv, 8 * inv], rtol=1e-7)
    X = np.random.default_rng(1).standard_normal((5, 300)).astype(np.float32)
    y = MR.rmsnorm(X, np.ones(300, np.float32), 0.0)
    assert np.allclose(np.sqrt((y.astype(np.float64) ** 2).mean(1)), 1.0, atol=1e-6)
    assert np.allclose(MR.rmsnorm(X[2], np.ones(300, np.float32), 0.0), y[2], rtol=1e-6)


def _attention_loops(q, K, V, hp, scale):
    group = hp.n_head // hp.n_kv
    out = np.zeros((hp.n_head, hp.head_dim))
    for h in range(hp.n_head):
        kvh = h // group
        s = [float(np.dot(q[h].astype(np.float64), K[t, kvh])) * scale for t in range(len(K))]
        m = max(s)
        e = [math.exp(v - m) for v in s]
        for t in range(len(K)):
            out[h] += e[t] / sum(e) * V[t, kvh]
    return out


def test_attention_matches_loops_and_closed_forms():
    hp = _hp(hd=8, n_head=4, n_kv=2)
    rng = np.random.default_rng(2)
    q = rng.standard_normal((4, 8)).astype(np.float32)
    K = rng.standard_normal((7, 2, 8)).astype(np.float32)
    V = rng.standard_normal((7, 2, 8)).astype(np.float32)
    got = MR.attention_np(q.reshape(-1), K, V, hp, 2, 0.35)
    assert np.allclose(got, _attention_loops(q, K, V, hp, 0.35), atol=1e-6)
    # one key: softmax weight 1, output = that value
    one = MR.attention_np(q.reshape(-1), K[:1], V[:1], hp, 2, 0.35)
    assert np.allclose(one, V[0][[0, 0, 1, 1]], atol=1e-7)
    # equal keys: the mean of the values
    Ke = np.repeat(K[:1], 7, axis=0)
    eq = MR.attention_np(q.reshape(-1), Ke, V, hp, 2, 0.35)
    assert np.allclose(eq, V.mean(0)[[0, 0, 1, 1]], atol=1e-6)
    # causal batch: row t attends to 0..t
    pos = np.arange(7, dtype=np.int32)
    qb = rng.standard_normal((7, 32)).astype(np.float32)
    bat = MR.attention_batch_np(qb, K, V, pos, hp, 2, 0.35)
    for t in range(7):
        ref = MR.attention_np(qb[t], K[:t + 1], V[:t + 1], hp, 2, 0.35)
        assert np.allclose(bat[t], ref.reshape(-1), atol=1e-6)


def test_forward_batch_equals_sequential(tiny):
    hp, tensors = tiny
    m = MR.RefModel(hp, tensors)
    toks = list(np.random.default_rng(4).integers(0, hp.n_vocab, 40))
    seq = [m.forward(t) for t in toks][-1]
    m.reset()
    bat = m.prefill(toks, chunk=16)  # three chunks, prefix reuse across chunks
    assert np.abs(seq - bat).max() < 1e-4  # tests/smoke.py:950-972


def test_forward_matches_pure_decoder(tiny):
    hp, tensors = tiny
    m = MR.RefModel(hp, tensors, fast=False)
    cache: dict = {}
    for t in (5, 77, 300):
        a = m.forward(t)
        b = m.forward_pure(t, cache)
        assert np.abs(a - b).max() < 1e-4 * max(1.0, np.abs(b).max())


def test_fast_loop_matches_einsum_path(tiny):
    hp, tensors = tiny
    a, b = MR.RefModel(hp, tensors, fast=True), MR.RefModel(hp, tensors, fast=False)
    for t in (1, 2, 3, 4):
        la, lb = a.forward(t), b.forward(t)
        assert np.abs(la - lb).max() < 1e-5 * np.abs(lb).max()


def test_planted_rope_mistake_is_caught(tiny, monkeypatch):
    """A sign error in the rotation must show up against the pure decoder."""
    hp, tensors = tiny
    good = MR.rope_np

    def bad(vec, n_heads, pos, hp_, cos, sin):
        return good(vec, n_heads, pos, hp_, cos, -sin)

    m = MR.RefModel(hp, tensors, fast=False)
    cache: dict = {}
    m.forward(9), m.forward_pure(9, cache)  # position 0: rotation is the identity
    monkeypatch.setattr(MR, "rope_np", bad)
    a, b = m.forward(10), m.forward_pure(10, cache)
    assert np.abs(a - b).max() > 1e-3 * np.abs(b).max()


def test_greedy_records_margins(tiny):
    hp, tensors = tiny
    m = MR.RefModel(hp, tensors)
    toks, margins = m.greedy([1, 2, 3], 6)
    assert len(toks) == 6 and len(margins) == 6 and min(margins) >= 0
    m.reset()
    assert toks[0] == int(np.argmax(m.prefill([1, 2, 3])))


def test_model_block_scales_pack_inverts_unpack():
    rng = np.random.default_rng(5)
    sc = rng.integers(0, 64, (1000, 8)).astype(np.uint8)
    mn = rng.integers(0, 64, (1000, 8)).astype(np.uint8)
    packed = synth.pack_kquant_scales(sc, mn)
    s2, m2 = Q.kquant_scales(packed)
    assert np.array_equal(s2, sc) and np.array_equal(m2, mn)


@pytest.mark.parametrize("dtype", ["Q4_K", "Q6_K"])
def test_model_blocks_zero_mean(dtype):
    b = synth.model_blocks(dtype, 256, 2048, seed=1, std=0.02)
    w = Q.dequantize(b.tobytes(), 256 * 2048, dtype).astype(np.float64)
    assert abs(w.mean()) < 0.05 * w.std()
    assert 0.015 < w.std() < 0.027
