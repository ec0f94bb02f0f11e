"""Oracle: the reference's decode step and greedy loop (TEST INFRASTRUCTURE -
see oracle/__init__.py).

A NumPy restatement of jtiro232/Alpacca alpacca/model.py over the
quantized-matrix oracle (qmatrix_ref.RefMatrix):

* ``RefModel.forward``       - Model.forward / _forward_np (model.py:436-441,
                               :520-555), float32 throughout;
* ``RefModel.forward_batch`` - Model.forward_batch (model.py:469-518): batched
                               prefill with causal attention;
* ``RefModel.prefill``       - Model.prefill (model.py:610-641), chunks of 256;
* ``RefModel.greedy``        - the greedy loop (tests/smoke.py:743-755):
                               logits = prefill(prompt), then argmax and
                               forward, recording the top-1/top-2 margins;
* ``RefModel.forward_pure``  - Model._forward_pure (model.py:557-608): Python
                               floats and explicit loops, an independent
                               restatement for tiny models;
* ``rmsnorm``, ``rope_np``, ``rope_batch_np``, ``attention_np``,
  ``attention_batch_np``, ``rope_tables`` - tensor.py:163-172,
  model.py:400-434, :447-467, :163-167 / :369-373.

Matvecs use RefMatrix.matvec_ref (qmatrix.py:160-171) or, with fast=True,
the C/OpenMP restatement of the reference's Numba loop (kernels.py:49-69);
prefill matmuls use RefMatrix.matmul_t_ref (qmatrix.py:196-211).

The model is described by duck-typed inputs: ``hp`` with the attributes of
the reference's Hyperparams (model.py:133-148) and ``tensors`` mapping GGUF
tensor names to objects with ``dtype``, ``shape`` and ``data``.
"""
from __future__ import annotations

import math

import numpy as np

from .quants_ref import DENSE_WIDTH, GEOMETRY
from .qmatrix_ref import DenseRef, RefMatrix


def rope_tables(hp, n_ctx: int):
    """model.py:163-167 (inv_freq) and :369-373 (tables)."""
    half = hp.n_rot // 2
    inv_freq = hp.rope_base ** (-2.0 * np.arange(half, dtype=np.float32) / hp.n_rot)
    theta = np.arange(n_ctx, dtype=np.float32)[:, None] * inv_freq[None, :]
    return np.cos(theta), np.sin(theta)


def rmsnorm(x, weight, eps: float):
    """tensor.py:163-172 (NumPy branch)."""
    arr = x if getattr(x, "dtype", None) == np.float32 else x.astype(np.float32)
    if arr.ndim == 1:
        inv = 1.0 / math.sqrt(float(arr @ arr) / arr.shape[0] + eps)
        return arr * inv * weight
    inv = 1.0 / np.sqrt(np.mean(arr * arr, axis=-1, keepdims=True) + eps)
    return arr * inv * weight


def rope_np(vec, n_heads: int, pos: int, hp, cos_t, sin_t):
    """model.py:400-416."""
    hd, n_rot = hp.head_dim, hp.n_rot
    half = n_rot // 2
    v = vec.reshape(n_heads, hd).copy()
    c, s = cos_t[pos], sin_t[pos]
    if hp.rope_style == "norm":
        x0 = v[:, 0:n_rot:2].copy()
        x1 = v[:, 1:n_rot:2].copy()
        v[:, 0:n_rot:2] = x0 * c - x1 * s
        v[:, 1:n_rot:2] = x0 * s + x1 * c
    else:
        x0 = v[:, :half].copy()
        x1 = v[:, half:n_rot].copy()
        v[:, :half] = x0 * c - x1 * s
        v[:, half:n_rot] = x0 * s + x1 * c
    return v.reshape(-1)


def rope_batch_np(vecs, n_heads: int, positions, hp, cos_t, sin_t):
    """model.py:418-434."""
    hd, n_rot = hp.head_dim, hp.n_rot
    half = n_rot // 2
    v = vecs.reshape(len(vecs), n_heads, hd).copy()
    c = cos_t[positions][:, None, :]
    s = sin_t[positions][:, None, :]
    if hp.rope_style == "norm":
        x0 = v[:, :, 0:n_rot:2].copy()
        x1 = v[:, :, 1:n_rot:2].copy()
        v[:, :, 0:n_rot:2] = x0 * c - x1 * s
        v[:, :, 1:n_rot:2] = x0 * s + x1 * c
    else:
        x0 = v[:, :, :half].copy()
        x1 = v[:, :, half:n_rot].copy()
        v[:, :, :half] = x0 * c - x1 * s
        v[:, :, half:n_rot] = x0 * s + x1 * c
    return v.reshape(len(vecs), -1)


def attention_np(q, K, V, hp, group: int, inv_sqrt: float):
    """model.py:447-455: q (n_head*hd), K/V (t, n_kv, hd)."""
    qg = q.reshape(hp.n_kv, group, hp.head_dim)
    scores = np.matmul(qg, K.transpose(1, 2, 0)) * inv_sqrt
    scores -= scores.max(axis=2, keepdims=True)
    w = np.exp(scores)
    w /= w.sum(axis=2, keepdims=True)
    att_out = np.matmul(w, V.transpose(1, 0, 2))
    return att_out.reshape(hp.n_head, hp.head_dim)


def attention_batch_np(q, K, V, positions, hp, group: int, inv_sqrt: float):
    """model.py:457-467: causal attention of a batch of queries."""
    qg = q.reshape(len(q), hp.n_kv, group, hp.head_dim)
    scores = np.einsum("tkgh,skh->tkgs", qg, K, optimize=True) * inv_sqrt
    allowed = np.arange(K.shape[0], dtype=np.int32)[None, :] <= positions[:, None]
    scores = np.where(allowed[:, None, None, :], scores, -1.0e30)
    scores -= scores.max(axis=-1, keepdims=True)
    w = np.exp(scores)
    w /= w.sum(axis=-1, keepdims=True)
    out = np.einsum("tkgs,skh->tkgh", w, V, optimize=True)
    return out.reshape(len(q), hp.n_head * hp.head_dim)


class _Mat:
    """A quantized matrix of the oracle: RefMatrix arithmetic, optionally the
    C restatement of the Numba loop for matvecs."""

    def __init__(self, t, fast: bool):
        rows, cols = t.shape
        self.rows, self.cols = rows, cols
        self._loop = None
        if t.dtype in DENSE_WIDTH:  # dense weights: NumPy products (model.py:276-281)
            self.ref = DenseRef(np.asarray(t.data).reshape(-1).view(np.uint8), t.dtype,
                                rows, cols)
            return
        self.ref = RefMatrix(t.data, t.dtype, rows, cols)
        if fast:
            from .cbaseline import LoopMatvec
            self._loop = LoopMatvec(self.ref.q3, self.ref.d, self.ref.m)

    def matvec(self, x):
        if self._loop is not None:
            return self._loop(np.asarray(x, dtype=np.float32))
        return self.ref.matvec_ref(x)

    def matmul_t(self, X):
        return self.ref.matmul_t_ref(X)

    def row(self, i: int):
        if not 0 <= i < self.rows:
            raise IndexError(i)
        return self.ref.rows_at([i])[0]

    def rows_at(self, idx):
        return self.ref.rows_at(idx)


class RefModel:
    def __init__(self, hp, tensors: dict, n_ctx: int = 0, fast: bool = True):
        self.hp = hp
        self.n_ctx = min(n_ctx, hp.n_ctx_train) if n_ctx else min(hp.n_ctx_train, 4096)

        def mat(name):
            return _Mat(tensors[name], fast)

        def vec(name):
            return np.asarray(tensors[name].data, dtype=np.float32).reshape(-1)

        self.tok_embd = mat("token_embd.weight")
        self.layers = []
        for i in range(hp.n_layer):
            p = f"blk.{i}."
            ly = {r: mat(p + r + ".weight") for r in
                  ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
                   "ffn_down")}
            ly["attn_norm"] = vec(p + "attn_norm.weight")
            ly["ffn_norm"] = vec(p + "ffn_norm.weight")
            for b in ("attn_q", "attn_k", "attn_v"):
                n = p + b + ".bias"
                ly[b + ".bias"] = vec(n) if n in tensors else None
            self.layers.append(ly)
        self.out_norm = vec("output_norm.weight")
        self.output = mat("output.weight") if "output.weight" in tensors else self.tok_embd
        self.cos, self.sin = rope_tables(hp, self.n_ctx)
        self.reset()

    def reset(self):
        hp = self.hp
        self.cache_k = [np.zeros((self.n_ctx, hp.n_kv, hp.head_dim), np.float32)
                        for _ in range(hp.n_layer)]
        self.cache_v = [np.zeros((self.n_ctx, hp.n_kv, hp.head_dim), np.float32)
                        for _ in range(hp.n_layer)]
        self.n_past = 0

    # model.py:436-441, :520-555
    def forward(self, token: int):
        hp = self.hp
        if self.n_past >= self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        pos = self.n_past
        x = self.tok_embd.row(token)
        inv_sqrt = 1.0 / math.sqrt(hp.head_dim)
        group = hp.n_head // hp.n_kv
        for li, ly in enumerate(self.layers):
            h = rmsnorm(x, ly["attn_norm"], hp.rms_eps)
            q = ly["attn_q"].matvec(h)
            k = ly["attn_k"].matvec(h)
            v = ly["attn_v"].matvec(h)
            if ly["attn_q.bias"] is not None:
                q = q + ly["attn_q.bias"]
            if ly["attn_k.bias"] is not None:
                k = k + ly["attn_k.bias"]
            if ly["attn_v.bias"] is not None:
                v = v + ly["attn_v.bias"]
            q = rope_np(q, hp.n_head, pos, hp, self.cos, self.sin).reshape(hp.n_head, hp.head_dim)
            k = rope_np(k, hp.n_kv, pos, hp, self.cos, self.sin).reshape(hp.n_kv, hp.head_dim)
            self.cache_k[li][pos] = k
            self.cache_v[li][pos] = v.reshape(hp.n_kv, hp.head_dim)
            K = self.cache_k[li][:pos + 1]
            V = self.cache_v[li][:pos + 1]
            att = attention_np(q, K, V, hp, group, inv_sqrt)
            x = x + ly["attn_output"].matvec(att.reshape(-1))
            h = rmsnorm(x, ly["ffn_norm"], hp.rms_eps)
            gate = ly["ffn_gate"].matvec(h)
            up = ly["ffn_up"].matvec(h)
            act = gate / (1.0 + np.exp(-gate)) * up
            x = x + ly["ffn_down"].matvec(act)
        self.n_past += 1
        return self.output.matvec(rmsnorm(x, self.out_norm, hp.rms_eps))

    # model.py:469-518
    def forward_batch(self, tokens):
        hp = self.hp
        if self.n_past + len(tokens) > self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        pos0 = self.n_past
        positions = np.arange(pos0, pos0 + len(tokens), dtype=np.int32)
        x = self.tok_embd.rows_at(tokens)
        inv_sqrt = 1.0 / math.sqrt(hp.head_dim)
        group = hp.n_head // hp.n_kv
        for li, ly in enumerate(self.layers):
            h = rmsnorm(x, ly["attn_norm"], hp.rms_eps)
            q = ly["attn_q"].matmul_t(h)
            k = ly["attn_k"].matmul_t(h)
            v = ly["attn_v"].matmul_t(h)
            if ly["attn_q.bias"] is not None:
                q = q + ly["attn_q.bias"]
            if ly["attn_k.bias"] is not None:
                k = k + ly["attn_k.bias"]
            if ly["attn_v.bias"] is not None:
                v = v + ly["attn_v.bias"]
            q = rope_batch_np(q, hp.n_head, positions, hp, self.cos, self.sin).reshape(
                len(tokens), hp.n_head, hp.head_dim)
            k = rope_batch_np(k, hp.n_kv, positions, hp, self.cos, self.sin).reshape(
                len(tokens), hp.n_kv, hp.head_dim)
            self.cache_k[li][pos0:pos0 + len(tokens)] = k
            self.cache_v[li][pos0:pos0 + len(tokens)] = v.reshape(len(tokens), hp.n_kv,
                                                                  hp.head_dim)
            K = self.cache_k[li][:pos0 + len(tokens)]
            V = self.cache_v[li][:pos0 + len(tokens)]
            att = attention_batch_np(q, K, V, positions, hp, group, inv_sqrt)
            x = x + ly["attn_output"].matmul_t(att)
            h = rmsnorm(x, ly["ffn_norm"], hp.rms_eps)
            gate = ly["ffn_gate"].matmul_t(h)
            up = ly["ffn_up"].matmul_t(h)
            act = gate / (1.0 + np.exp(-gate)) * up
            x = x + ly["ffn_down"].matmul_t(act)
        self.n_past += len(tokens)
        return self.output.matvec(rmsnorm(x[-1], self.out_norm, self.hp.rms_eps))

    # model.py:610-641 (from an empty cache; chunks of ALPACCA_PREFILL_CHUNK=256)
    def prefill(self, tokens, chunk: int = 256):
        logits = None
        for i in range(0, len(tokens), chunk):
            logits = self.forward_batch(tokens[i:i + chunk])
        return logits

    def greedy(self, prompt, n_gen: int, chunk: int = 256, progress=None,
               repeat_penalty: float = 1.0, repeat_last_n: int = 64):
        """n_gen greedy tokens after prompt (smoke.py:743-755 with plain
        argmax, tensor.py:187-194).  Returns (tokens, margins): margin i is
        the gap between the largest and second-largest logit at step i.
        With repeat_penalty not 0 or 1 it is the decode loop of
        tests/bench.py:78-90: a Sampler at temperature 0 that accepts the
        prompt, then each chosen token, and penalizes the last repeat_last_n
        (sample.py:31-45); margins are then of the penalized values."""
        from .sample_ref import RepeatWindow, penalized_argmax, penalized_margin
        self.reset()
        window = RepeatWindow(repeat_last_n)
        for t in prompt:
            window.accept(t)
        logits = self.prefill(list(prompt), chunk)
        toks, margins = [], []
        for i in range(n_gen):
            t = penalized_argmax(logits, window.recent, repeat_penalty)
            toks.append(t)
            margins.append(penalized_margin(logits, window.recent, repeat_penalty))
            window.accept(t)
            if progress:
                progress(i, t)
            if i + 1 < n_gen:
                logits = self.forward(t)
        return toks, margins

    # model.py:557-608: the pure-Python decoder, for tiny models
    def forward_pure(self, token: int, cache: dict):
        hp = self.hp
        pos = cache.setdefault("n_past", 0)
        hd = hp.head_dim
        group = hp.n_head // hp.n_kv
        inv_sqrt = 1.0 / math.sqrt(hd)

        def mv(m, v):
            W = m.ref.dense().astype(np.float64)
            return [float(sum(W[r, c] * v[c] for c in range(m.cols))) for r in range(m.rows)]

        def norm(v, w):
            ss = sum(a * a for a in v) / len(v)
            inv = 1.0 / math.sqrt(ss + hp.rms_eps)
            return [a * inv * float(b) for a, b in zip(v, w)]

        def rope(vec, n_heads):
            out = list(vec)
            half = hp.n_rot // 2
            for h in range(n_heads):
                base = h * hd
                for i in range(half):
                    theta = pos * hp.rope_base ** (-2.0 * i / hp.n_rot)
                    c, s = math.cos(theta), math.sin(theta)
                    if hp.rope_style == "norm":
                        a, b = base + 2 * i, base + 2 * i + 1
                    else:
                        a, b = base + i, base + half + i
                    x0, x1 = out[a], out[b]
                    out[a] = x0 * c - x1 * s
                    out[b] = x0 * s + x1 * c
            return out

        x = [float(v) for v in self.tok_embd.row(token)]
        for li, ly in enumerate(self.layers):
            h = norm(x, ly["attn_norm"])
            q, k, v = mv(ly["attn_q"], h), mv(ly["attn_k"], h), mv(ly["attn_v"], h)
            for b, vecv in (("attn_q", q), ("attn_k", k), ("attn_v", v)):
                if ly[b + ".bias"] is not None:
                    for i, bv in enumerate(ly[b + ".bias"]):
                        vecv[i] += float(bv)
            q, k = rope(q, hp.n_head), rope(k, hp.n_kv)
            cache.setdefault(("k", li), []).append(k)
            cache.setdefault(("v", li), []).append(v)
            att = [0.0] * (hp.n_head * hd)
            for hh in range(hp.n_head):
                kvh = hh // group
                qh = q[hh * hd:(hh + 1) * hd]
                scores = [sum(a * b for a, b in zip(qh, kt[kvh * hd:(kvh + 1) * hd])) * inv_sqrt
                          for kt in cache[("k", li)]]
                m = max(scores)
                e = [math.exp(s - m) for s in scores]
                tot = sum(e)
                for t, wt in enumerate(e):
                    vt = cache[("v", li)][t][kvh * hd:(kvh + 1) * hd]
                    for d in range(hd):
                        att[hh * hd + d] += wt / tot * vt[d]
            x = [a + b for a, b in zip(x, mv(ly["attn_output"], att))]
            h = norm(x, ly["ffn_norm"])
            g, u = mv(ly["ffn_gate"], h), mv(ly["ffn_up"], h)
            act = [(gv / (1.0 + math.exp(-gv)) if gv >= 0 else gv * math.exp(gv) / (1.0 + math.exp(gv))) * uv
                   for gv, uv in zip(g, u)]
            x = [a + b for a, b in zip(x, mv(ly["ffn_down"], act))]
        cache["n_past"] = pos + 1
        return np.array(mv(self.output, norm(x, self.out_norm)))


def model_weight_bytes(tensors: dict, names) -> int:
    """Raw GGUF bytes of the named quantized tensors."""
    total = 0
    for n in names:
        t = tensors[n]
        if t.dtype in DENSE_WIDTH:
            total += t.shape[0] * t.shape[1] * DENSE_WIDTH[t.dtype]
            continue
        be, bb, _, _ = GEOMETRY[t.dtype]
        total += t.shape[0] * (t.shape[1] // be) * bb
    return total
