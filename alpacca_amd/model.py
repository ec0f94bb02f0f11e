"""Device-resident decode of a llama-family model whose linear layers are
QuantMatrix objects: the callers of the quantized matvec in the reference's
decode step (alpacca/model.py:520-555, Model._forward_np) and its greedy
loop, run on one GPU through the C ABI of libalpacca_amd.so.

Mirrors the reference's ``Model`` where it touches the hot path:

* ``forward(token)`` - one token at position ``n_past``; returns the logits
  (model.py:436-441 / :520-555);
* ``prefill(tokens)`` - feeds a prompt; returns the last token's logits
  (model.py:610-641; prompt tokens run through the decode step one by one,
  which computes the same function as the reference's chunked forward_batch);
* ``generate_greedy(prompt, n)`` - ``n`` greedy tokens after the prompt
  (argmax of the logits, tensor.py:187-194, fed back as the next token).

Layer weights, KV cache, activations, position and token all stay in HBM.
One decode step is a fixed sequence of kernel launches that reads the token
and position from a device-side ``aq_decode_state``, so ``generate_greedy``
captures it once as a HIP graph and replays it per token with no host work
in between.

Buffers are PyTorch CUDA tensors (plumbing only); all compute is in the HIP
library, and a missing library or GPU raises instead of falling back.
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass

import numpy as np

from . import _lib
from .qmatrix import (DENSE_DTYPES, MIXABLE_DTYPES, DenseMatrix, QuantMatrix,
                      interleave_rows, matvec_fused_device, matvec_multi_device,
                      pair_rows_supported)

ROPE_STYLES = {"llama": "norm", "mistral": "norm", "qwen2": "neox", "qwen3": "neox",
               "stablelm": "neox", "gemma": "neox"}  # model.py:22-29


@dataclass
class Hyperparams:
    """The reference's Hyperparams (alpacca/model.py:133-148)."""
    arch: str
    n_layer: int
    n_embd: int
    n_head: int
    n_kv: int
    n_ff: int
    n_vocab: int
    n_ctx_train: int
    head_dim: int
    n_rot: int
    rms_eps: float
    rope_base: float
    rope_style: str


@dataclass
class Tensor:
    """A named weight: quantized GGUF blocks (dtype, rows x cols) or a dense
    float32 vector (dtype "F32", e.g. the norm weights)."""
    dtype: str
    shape: tuple
    data: object  # bytes-like blocks, or a float32 ndarray for F32


LAYER_ROLES = ("attn_q", "attn_k", "attn_v", "attn_output", "ffn_gate", "ffn_up",
               "ffn_down")


def rope_tables(hp: Hyperparams, n_ctx: int) -> tuple[np.ndarray, np.ndarray]:
    """float32 cos/sin of pos * inv_freq, (n_ctx, n_rot/2), computed exactly as
    the reference computes them (model.py:163-167, :369-373)."""
    half = hp.n_rot // 2
    inv_freq = hp.rope_base ** (-2.0 * np.arange(half, dtype=np.float32) / hp.n_rot)
    theta = np.arange(n_ctx, dtype=np.float32)[:, None] * inv_freq[None, :]
    return np.cos(theta), np.sin(theta)


class Model:
    """Greedy decode of a model given as a dict of Tensors (GGUF names)."""

    def __init__(self, hp: Hyperparams, tensors: dict, n_ctx: int = 0, layout=None,
                 fused: bool = True):
        import torch
        if not torch.cuda.is_available():
            raise RuntimeError("alpacca_amd.model.Model needs a HIP device (gfx950)")
        _lib.ensure_device()
        self.torch = torch
        self.hp = hp
        # fused=True folds RMSNorm, SwiGLU and the residual adds into the
        # matvec launches (aq_matvec_fused); False runs them as separate kernels
        self.fused = fused
        self.dev = torch.device("cuda", torch.cuda.current_device())
        # model.py:332: the context defaults to min(n_ctx_train, 4096)
        self.n_ctx = min(n_ctx, hp.n_ctx_train) if n_ctx else min(hp.n_ctx_train, 4096)
        self.stream = torch.cuda.Stream(self.dev)  # default priority
        q_dim, kv_dim = hp.n_head * hp.head_dim, hp.n_kv * hp.head_dim
        if hp.n_rot > hp.head_dim or hp.n_rot % 2:
            raise ValueError("n_rot must be even and at most head_dim")

        def mat(name, rows, cols):
            t = tensors.get(name)
            if t is None:
                raise ValueError(f"missing tensor {name}")
            if tuple(t.shape) != (rows, cols):
                raise ValueError(f"tensor {name} has shape {t.shape}, expected {(rows, cols)}")
            if t.dtype in DENSE_DTYPES:  # the reference's dense matrices (model.py:276-281)
                return DenseMatrix(t.data, t.dtype, rows, cols)
            return QuantMatrix(t.data, t.dtype, rows, cols, layout=layout)

        def vec(name, n):
            t = tensors.get(name)
            if t is None:
                raise ValueError(f"missing tensor {name}")
            v = np.asarray(t.data, dtype=np.float32).reshape(-1)
            if v.size != n:
                raise ValueError(f"tensor {name} has {v.size} elements, expected {n}")
            return torch.from_numpy(v.copy()).to(self.dev)

        self.tok_embd = mat("token_embd.weight", hp.n_vocab, hp.n_embd)
        self.layers = []
        for i in range(hp.n_layer):
            p = f"blk.{i}."
            ly = {
                "attn_norm": vec(p + "attn_norm.weight", hp.n_embd),
                "ffn_norm": vec(p + "ffn_norm.weight", hp.n_embd),
                "attn_q": mat(p + "attn_q.weight", q_dim, hp.n_embd),
                "attn_k": mat(p + "attn_k.weight", kv_dim, hp.n_embd),
                "attn_v": mat(p + "attn_v.weight", kv_dim, hp.n_embd),
                "attn_output": mat(p + "attn_output.weight", hp.n_embd, q_dim),
                "ffn_gate": mat(p + "ffn_gate.weight", hp.n_ff, hp.n_embd),
                "ffn_up": mat(p + "ffn_up.weight", hp.n_ff, hp.n_embd),
                "ffn_down": mat(p + "ffn_down.weight", hp.n_embd, hp.n_ff),
            }
            for b in ("attn_q", "attn_k", "attn_v"):  # optional biases (qwen2)
                t = tensors.get(p + b + ".bias")
                ly[b + ".bias"] = None if t is None else vec(p + b + ".bias", ly[b].rows)
            # fused step: gate and up rows interleaved in one matrix, so the
            # gate/up launch writes silu(gate) * up itself (row pairs) and
            # ffn_down reads plain x; the batched prefill multiplies the same
            # matrix and takes SwiGLU over the pairs, so the separate matrices
            # are dropped below unless the unfused step needs them
            g, u = tensors[p + "ffn_gate.weight"], tensors[p + "ffn_up.weight"]
            ly["ffn_gate_up"] = None
            if (fused and g.dtype == u.dtype and isinstance(ly["ffn_gate"], QuantMatrix)
                    and ly["ffn_gate"].layout == ly["ffn_up"].layout
                    and pair_rows_supported(g.dtype, hp.n_embd)):
                ly["ffn_gate_up"] = QuantMatrix(
                    interleave_rows(g.data, u.data, hp.n_ff, hp.n_embd, g.dtype), g.dtype,
                    2 * hp.n_ff, hp.n_embd, layout=ly["ffn_gate"].layout)
            self.layers.append(ly)
        self.out_norm = vec("output_norm.weight", hp.n_embd)
        self.output = (mat("output.weight", hp.n_vocab, hp.n_embd)
                       if "output.weight" in tensors else self.tok_embd)  # tied
        # dense matrices have no fused launches: such a model runs the
        # unfused step (RMSNorm, SwiGLU and adds as their own kernels)
        if any(isinstance(m, DenseMatrix) for ly in self.layers for m in ly.values()) or \
                isinstance(self.output, DenseMatrix):
            self.fused = False
        # one copy of gate/up in HBM: the interleaved matrix when the fused
        # step uses it, the separate ones otherwise
        for ly in self.layers:
            if ly["ffn_gate_up"] is None:
                continue
            if self.fused:
                ly["ffn_gate"] = ly["ffn_up"] = None
            else:
                ly["ffn_gate_up"] = None

        f32 = dict(dtype=torch.float32, device=self.dev)
        cos, sin = rope_tables(hp, self.n_ctx)
        self.rope_cos = torch.from_numpy(np.ascontiguousarray(cos)).to(self.dev)
        self.rope_sin = torch.from_numpy(np.ascontiguousarray(sin)).to(self.dev)
        self.kv = torch.zeros((hp.n_layer, 2, hp.n_kv, self.n_ctx, hp.head_dim), **f32)
        self.x = torch.zeros(hp.n_embd, **f32)
        self.h = torch.zeros(hp.n_embd, **f32)
        self.o = torch.zeros(hp.n_embd, **f32)
        self.q = torch.zeros(q_dim, **f32)
        self.k = torch.zeros(kv_dim, **f32)
        self.v = torch.zeros(kv_dim, **f32)
        self.att = torch.zeros(q_dim, **f32)
        self.gate = torch.zeros(hp.n_ff, **f32)
        self.up = torch.zeros(hp.n_ff, **f32)
        self.act = torch.zeros(hp.n_ff, **f32)
        self.logits = torch.zeros(hp.n_vocab, **f32)
        # aq_decode_state: int64 token, uint64 key, int32 pos, fed, count, pad
        self.state = torch.zeros(_lib.DECODE_STATE_BYTES // 4, dtype=torch.int32,
                                 device=self.dev)
        self.n_past = 0
        self.cached_ids: list[int] = []
        # batched prefill: chunk size (ALPACCA_PREFILL_CHUNK, model.py:630-634)
        # and matmul precision (fp32 MFMA: the reference's f32 products).  The
        # reference's 256 bounds host memory; here the chunk only sets how
        # many rows each matmul_t launch gets (the results are bit-identical
        # for every chunk size: a product's K order does not depend on M and
        # attention merges fixed 64-position chunks), and 256-row launches
        # leave most CUs idle (1B model, 2048 tokens: 298 ms at 256, 70 ms
        # at 2048).
        import os
        try:
            self.prefill_chunk = max(1, int(os.environ.get("ALPACCA_PREFILL_CHUNK", "2048")))
        except ValueError:
            self.prefill_chunk = 2048
        self.prefill_precision = "fp32"

    # ---- state ------------------------------------------------------------

    def _set_state(self, token: int, pos: int, fed: int = 0, count: int = 0) -> None:
        st = np.zeros(_lib.DECODE_STATE_BYTES // 4, dtype=np.int32)
        st[0:2] = np.array([token], dtype=np.int64).view(np.int32)
        st[4], st[5], st[6] = pos, fed, count  # key and done stay 0
        self.state.copy_(self.torch.from_numpy(st))

    def reset(self) -> None:
        """Empty the KV cache (model.py:375-376)."""
        self.n_past = 0
        self.cached_ids = []

    # ---- one step, enqueued on self.stream ---------------------------------

    def _enqueue_layers(self) -> None:
        hp, lib, s = self.hp, _lib.load(), self.stream.cuda_stream
        st = self.state.data_ptr()
        chk = _lib.check
        # x = token_embd[state.token] (the token is the state's first field)
        self.tok_embd.rows_at_device(st, 1, self.x.data_ptr(), s)
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        sv = ctypes.c_void_p(s)
        for li, ly in enumerate(self.layers):
            kc, vc = self.kv[li, 0], self.kv[li, 1]
            if self.fused:
                self._matvecs([ly["attn_q"], ly["attn_k"], ly["attn_v"]],
                              [self.q, self.k, self.v], self.x, s, norm=ly["attn_norm"])
            else:
                chk(lib.aq_rmsnorm(p(self.x), p(ly["attn_norm"]), 1, hp.n_embd,
                                   ctypes.c_float(hp.rms_eps), p(self.h), sv))
                self._matvecs([ly["attn_q"], ly["attn_k"], ly["attn_v"]],
                              [self.q, self.k, self.v], self.h, s)
            for b, out in (("attn_q", self.q), ("attn_k", self.k), ("attn_v", self.v)):
                if ly[b + ".bias"] is not None:
                    chk(lib.aq_add(p(out), p(ly[b + ".bias"]), out.numel(), sv))
            neox = 1 if hp.rope_style == "neox" else 0
            if self.fused and not (neox and hp.n_rot % 8):
                chk(lib.aq_attention_rope(p(self.q), p(self.k), p(self.v), hp.n_head, hp.n_kv,
                                          hp.head_dim, hp.n_rot, neox, p(self.rope_cos),
                                          p(self.rope_sin), ctypes.c_void_p(st), 0,
                                          self.n_ctx, p(kc), p(vc), p(self.att), sv))
            else:
                chk(lib.aq_rope_kv(p(self.q), p(self.k), p(self.v), 1, hp.n_head, hp.n_kv,
                                   hp.head_dim, hp.n_rot, neox, p(self.rope_cos),
                                   p(self.rope_sin), ctypes.c_void_p(st), 0, self.n_ctx,
                                   p(kc), p(vc), sv))
                chk(lib.aq_attention(p(self.q), p(kc), p(vc), hp.n_head, hp.n_kv,
                                     hp.head_dim, self.n_ctx, ctypes.c_void_p(st), 0,
                                     p(self.att), sv))
            if self.fused:
                matvec_fused_device([ly["attn_output"]], self.att.data_ptr(),
                                    [self.x.data_ptr()], s, accumulate=True)
                if ly["ffn_gate_up"] is not None:  # SwiGLU in the gate/up store
                    matvec_fused_device([ly["ffn_gate_up"]], self.x.data_ptr(),
                                        [self.act.data_ptr()], s,
                                        norm_w_ptr=ly["ffn_norm"].data_ptr(),
                                        eps=hp.rms_eps, rmsnorm=True, swiglu_pairs=True)
                    matvec_fused_device([ly["ffn_down"]], self.act.data_ptr(),
                                        [self.x.data_ptr()], s, accumulate=True)
                    continue
                self._matvecs([ly["ffn_gate"], ly["ffn_up"]], [self.gate, self.up], self.x, s,
                              norm=ly["ffn_norm"])
                matvec_fused_device([ly["ffn_down"]], self.gate.data_ptr(), [self.x.data_ptr()],
                                    s, x2_ptr=self.up.data_ptr(), swiglu=True, accumulate=True)
                continue
            ly["attn_output"].matvec_device(self.att.data_ptr(), self.o.data_ptr(), s)
            chk(lib.aq_add(p(self.x), p(self.o), hp.n_embd, sv))
            chk(lib.aq_rmsnorm(p(self.x), p(ly["ffn_norm"]), 1, hp.n_embd,
                               ctypes.c_float(hp.rms_eps), p(self.h), sv))
            self._matvecs([ly["ffn_gate"], ly["ffn_up"]], [self.gate, self.up], self.h, s)
            chk(lib.aq_swiglu(p(self.gate), p(self.up), hp.n_ff, p(self.act), sv))
            ly["ffn_down"].matvec_device(self.act.data_ptr(), self.o.data_ptr(), s)
            chk(lib.aq_add(p(self.x), p(self.o), hp.n_embd, sv))

    def _matvecs(self, mats, outs, x, s, norm=None) -> None:
        """Matrices that share x and agree in dtype and K run as one launch
        (two dtypes of MIXABLE_DTYPES too: q/k in Q4_K with v in Q6_K); with
        `norm`, the launch applies RMSNorm(x) * norm itself."""
        groups: dict = {}
        for m, y in zip(mats, outs):
            groups.setdefault((m.dtype, m.cols, m.layout), []).append((m, y))
        keys = list(groups)
        if (len(keys) == 2 and keys[0][1] == keys[1][1]
                and (keys[0][0], keys[1][0]) in MIXABLE_DTYPES):
            groups = {tuple(keys): groups[keys[0]] + groups[keys[1]]}
        for grp in groups.values():
            ms, ys = [m for m, _ in grp], [y.data_ptr() for _, y in grp]
            if isinstance(ms[0], DenseMatrix):  # one fp32-kernel launch each
                for m, y in zip(ms, ys):
                    m.matvec_device(x.data_ptr(), y, s)
                continue
            if norm is not None:
                matvec_fused_device(ms, x.data_ptr(), ys, s, norm_w_ptr=norm.data_ptr(),
                                    eps=self.hp.rms_eps, rmsnorm=True)
            elif len(grp) == 1:
                ms[0].matvec_device(x.data_ptr(), ys[0], s)
            else:
                matvec_multi_device(ms, x.data_ptr(), ys, s)

    def _enqueue_head(self) -> None:
        hp, lib, s = self.hp, _lib.load(), self.stream.cuda_stream
        if self.fused:
            self._matvecs([self.output], [self.logits], self.x, s, norm=self.out_norm)
            return
        _lib.check(lib.aq_rmsnorm(ctypes.c_void_p(self.x.data_ptr()),
                                  ctypes.c_void_p(self.out_norm.data_ptr()), 1, hp.n_embd,
                                  ctypes.c_float(hp.rms_eps),
                                  ctypes.c_void_p(self.h.data_ptr()), ctypes.c_void_p(s)))
        self.output.matvec_device(self.h.data_ptr(), self.logits.data_ptr(), s)

    def _enqueue_advance(self, take_argmax: bool, prompt=None, hist=None,
                         window=None, penalty: float = 1.0) -> None:
        """End of step: pos += 1; the next token is the next prompt token
        while any is left, else (take_argmax) the argmax of the logits -
        with `window` (device int64 [1 + last_n]: count, ring of the
        accepted tokens) the argmax after the repetition penalty."""
        lib, s = _lib.load(), self.stream.cuda_stream
        args = (ctypes.c_void_p(self.logits.data_ptr()), self.hp.n_vocab,
                ctypes.c_void_p(self.state.data_ptr()),
                ctypes.c_void_p(prompt.data_ptr() if prompt is not None else 0),
                prompt.numel() if prompt is not None else 0,
                ctypes.c_void_p(hist.data_ptr() if hist is not None else 0),
                hist.numel() if hist is not None else 0)
        if window is None:
            _lib.check(lib.aq_greedy_advance(*args, 1 if take_argmax else 0,
                                             ctypes.c_void_p(s)))
        else:
            _lib.check(lib.aq_greedy_advance_penalized(
                *args, ctypes.c_void_p(window.data_ptr()), window.numel() - 1,
                ctypes.c_double(penalty), 1 if take_argmax else 0, ctypes.c_void_p(s)))

    # ---- the reference's entry points ---------------------------------------

    def forward(self, token: int) -> np.ndarray:
        """Process one token at position n_past; returns its logits
        (model.py:436-441)."""
        if self.n_past >= self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        if not 0 <= token < self.hp.n_vocab:
            raise IndexError("row index out of range")
        torch = self.torch
        with torch.cuda.stream(self.stream):
            self._set_state(token, self.n_past)
            self._enqueue_layers()
            self._enqueue_head()
            self._enqueue_advance(False)
        self.stream.synchronize()
        self.n_past += 1
        self.cached_ids.append(token)
        return self.logits.cpu().numpy()

    def prefill(self, tokens: list[int], batch: bool = True):
        """Feed prompt tokens; returns the logits of the last one
        (model.py:610-641).  Positions continue from n_past; a prompt that
        repeats the cached prefix reuses it as the reference does.  batch=True
        runs the suffix through the batched step (forward_batch, in chunks of
        prefill_chunk tokens); batch=False runs it through the decode step
        one token at a time (the same function)."""
        if not tokens:
            return None
        if len(tokens) > self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        n = 0
        max_prefix = min(len(tokens), len(self.cached_ids))
        while n < max_prefix and tokens[n] == self.cached_ids[n]:
            n += 1
        if n == len(tokens):
            n = max(0, len(tokens) - 1)
        if n != self.n_past:
            n = min(n, self.n_past)
            self.n_past = n
            del self.cached_ids[n:]
        suffix = list(tokens[n:])
        if batch:
            return self._prefill_batch(suffix)
        self._run_prompt(suffix[:-1])
        return self.forward(suffix[-1])

    # ---- batched prefill (Model.forward_batch, model.py:469-518) ------------

    def _batch_buffers(self, T: int) -> dict:
        b = getattr(self, "_bb", None)
        if b is None or b["T"] < T:
            torch, hp = self.torch, self.hp
            f32 = dict(dtype=torch.float32, device=self.dev)
            q_dim, kv_dim = hp.n_head * hp.head_dim, hp.n_kv * hp.head_dim
            # GU: T x 2 n_ff, the interleaved gate/up products, or G and U
            # (T x n_ff each) as its two halves for separate matrices
            gu = torch.zeros(2 * T * hp.n_ff, **f32)
            b = {"T": T, "ids": torch.zeros(T, dtype=torch.int64, device=self.dev),
                 "X": torch.zeros((T, hp.n_embd), **f32), "H": torch.zeros((T, hp.n_embd), **f32),
                 "O": torch.zeros((T, hp.n_embd), **f32), "Q": torch.zeros((T, q_dim), **f32),
                 "K": torch.zeros((T, kv_dim), **f32), "V": torch.zeros((T, kv_dim), **f32),
                 "A": torch.zeros((T, q_dim), **f32), "GU": gu.view(T, 2 * hp.n_ff),
                 "G": gu[:T * hp.n_ff].view(T, hp.n_ff), "U": gu[T * hp.n_ff:].view(T, hp.n_ff),
                 "S": torch.zeros((T, hp.n_ff), **f32)}
            self._bb = b
        return b

    def _prefill_batch(self, tokens: list[int]) -> np.ndarray:
        """The batched step over chunks of prefill_chunk tokens at positions
        n_past..: RMSNorm of all rows, matmul_t for every projection (fp32
        MFMA unless prefill_precision says otherwise), RoPE + KV store of the
        chunk, causal attention of its queries, SwiGLU, residual adds; then
        the head on the last token only.  Returns its logits."""
        hp, torch = self.hp, self.torch
        if self.n_past + len(tokens) > self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        if min(tokens) < 0 or max(tokens) >= hp.n_vocab:
            raise IndexError("row index out of range")
        lib, s = _lib.load(), self.stream.cuda_stream
        sv, chk = ctypes.c_void_p(s), _lib.check
        p = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        prec = self.prefill_precision
        neox = 1 if hp.rope_style == "neox" else 0
        chunk = self.prefill_chunk
        b = self._batch_buffers(min(chunk, len(tokens)))
        X, H, O, Q, K, V, A, G, U, S = (b[k] for k in "XHOQKVAGUS")
        GU = b["GU"]
        eps, n_layers = ctypes.c_float(hp.rms_eps), len(self.layers)
        with torch.cuda.stream(self.stream):
            for c0 in range(0, len(tokens), chunk):
                toks = tokens[c0:c0 + chunk]
                T, pos0 = len(toks), self.n_past
                b["ids"][:T].copy_(torch.tensor(toks, dtype=torch.int64))
                self.tok_embd.rows_at_device(b["ids"].data_ptr(), T, X.data_ptr(), s)
                # the first RMSNorm on its own; each later one shares a launch
                # with the residual add before it (aq_add_rmsnorm, the same bits)
                chk(lib.aq_rmsnorm(p(X), p(self.layers[0]["attn_norm"]), T, hp.n_embd, eps,
                                   p(H), sv))
                for li, ly in enumerate(self.layers):
                    kc, vc = self.kv[li, 0], self.kv[li, 1]
                    for role, out in (("attn_q", Q), ("attn_k", K), ("attn_v", V)):
                        ly[role].matmul_t_device(H.data_ptr(), T, out.data_ptr(), s, prec)
                        if ly[role + ".bias"] is not None:  # q + bq over the batch
                            chk(lib.aq_add_rows(p(out), p(ly[role + ".bias"]), T,
                                                out.shape[1], sv))
                    chk(lib.aq_rope_kv(p(Q), p(K), p(V), T, hp.n_head, hp.n_kv, hp.head_dim,
                                       hp.n_rot, neox, p(self.rope_cos), p(self.rope_sin),
                                       None, pos0, self.n_ctx, p(kc), p(vc), sv))
                    chk(lib.aq_attention_batch(p(Q), p(kc), p(vc), T, hp.n_head, hp.n_kv,
                                               hp.head_dim, self.n_ctx, None, pos0, p(A), sv))
                    ly["attn_output"].matmul_t_device(A.data_ptr(), T, O.data_ptr(), s, prec)
                    chk(lib.aq_add_rmsnorm(p(X), p(O), p(ly["ffn_norm"]), T, hp.n_embd, eps,
                                           p(H), sv))
                    if ly["ffn_gate_up"] is not None:  # (gate, up) pairs from one product
                        ly["ffn_gate_up"].matmul_t_swiglu_device(H.data_ptr(), T, GU.data_ptr(),
                                                                 S.data_ptr(), s, prec)
                    else:
                        ly["ffn_gate"].matmul_t_device(H.data_ptr(), T, G.data_ptr(), s, prec)
                        ly["ffn_up"].matmul_t_device(H.data_ptr(), T, U.data_ptr(), s, prec)
                        chk(lib.aq_swiglu(p(G), p(U), T * hp.n_ff, p(S), sv))
                    ly["ffn_down"].matmul_t_device(S.data_ptr(), T, O.data_ptr(), s, prec)
                    if li + 1 < n_layers:
                        chk(lib.aq_add_rmsnorm(p(X), p(O), p(self.layers[li + 1]["attn_norm"]),
                                               T, hp.n_embd, eps, p(H), sv))
                    else:
                        chk(lib.aq_add(p(X), p(O), T * hp.n_embd, sv))
                self.n_past += T
            self.x.copy_(X[T - 1])
            self._enqueue_head()
        self.stream.synchronize()
        self.cached_ids.extend(tokens)
        return self.logits.cpu().numpy()

    def _run_prompt(self, tokens: list[int]) -> None:
        """Run tokens through the decode step (KV cache only, no logits)."""
        if not tokens:
            return
        if self.n_past + len(tokens) > self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        if min(tokens) < 0 or max(tokens) >= self.hp.n_vocab:
            raise IndexError("row index out of range")
        torch = self.torch
        prompt = torch.tensor(tokens, dtype=torch.int64, device=self.dev)
        with torch.cuda.stream(self.stream):
            self._set_state(tokens[0], self.n_past, fed=1)
            for _ in tokens:
                self._enqueue_layers()
                self._enqueue_advance(False, prompt)
        self.stream.synchronize()
        self.n_past += len(tokens)
        self.cached_ids.extend(tokens)

    def generate_greedy(self, prompt: list[int], n_gen: int, graph: bool = True,
                        timing: dict | None = None, batch_prefill: bool = True,
                        repeat_penalty: float = 1.0, repeat_last_n: int = 64,
                        steps_per_graph: int = 16) -> list[int]:
        """Greedy continuation: n_gen tokens after `prompt` (the loop of
        smoke.py:743-755: logits = prefill(prompt); token = argmax(logits);
        logits = forward(token) ...).  Starts from an empty cache.  The
        prompt runs through the batched step (batch_prefill=True) or through
        the decode step; every generated token after the first is one decode
        step.  With graph=True the steps run as HIP graph replays of
        steps_per_graph steps each (the state advances on the device, so the
        steps are identical; one replay of a one-step graph per token for the
        remainder): 1807-1815 tok/s on the 1B model at 8-64 steps per graph
        against 1791-1793 at one.  `timing`, if given,
        receives the elapsed milliseconds of those n_gen - 1 decode steps
        (HIP events on the launch stream), their count, and the wall time of
        the prompt (prefill_ms).

        repeat_penalty other than 0 and 1 gives the decode loop of
        tests/bench.py:78-90 instead: a temperature-0 Sampler that accepts
        the prompt and every chosen token and penalizes the last
        max(repeat_last_n, 1) of them (sample.py:31-45), on the device."""
        torch = self.torch
        if not prompt or n_gen < 1:
            raise ValueError("need a non-empty prompt and n_gen >= 1")
        penalize = bool(repeat_penalty) and repeat_penalty != 1.0
        if penalize and not np.isfinite(repeat_penalty):
            raise ValueError("repeat_penalty must be finite")
        if len(prompt) + n_gen - 1 > self.n_ctx:
            raise RuntimeError(f"context window full ({self.n_ctx} tokens)")
        if min(prompt) < 0 or max(prompt) >= self.hp.n_vocab:
            raise IndexError("row index out of range")
        self.reset()
        prompt_dev = torch.tensor(prompt, dtype=torch.int64, device=self.dev)
        hist = torch.zeros(n_gen, dtype=torch.int64, device=self.dev)
        n_p = len(prompt)
        window = None
        if penalize:  # Sampler.accept of the prompt (tests/bench.py:78-80)
            last_n = max(int(repeat_last_n), 1)
            ring = np.zeros(1 + last_n, dtype=np.int64)
            for i, t in enumerate(prompt):
                ring[1 + i % last_n] = t
            ring[0] = n_p
            window = torch.zeros(1 + last_n, dtype=torch.int64, device=self.dev)

        def advance():
            self._enqueue_advance(True, None, hist, window, repeat_penalty)

        def prompt_step():
            self._enqueue_layers()
            self._enqueue_advance(False, prompt_dev)

        def gen_step():
            self._enqueue_layers()
            self._enqueue_head()
            advance()

        per_graph = max(1, int(steps_per_graph))
        run_prompt, run_gen, run_gen_k = prompt_step, gen_step, None
        if graph:  # captured first: the captures' eager warmup steps write junk
            g_gen = self._capture(gen_step)  # that the prompt then overwrites
            run_gen = g_gen.replay
            if per_graph > 1 and n_gen - 1 >= per_graph:
                def gen_k():
                    for _ in range(per_graph):
                        gen_step()
                run_gen_k = self._capture(gen_k).replay
            if not batch_prefill:
                with torch.cuda.stream(self.stream):
                    self._set_state(prompt[0], 0, fed=1)
                g_prompt = self._capture(prompt_step)
                run_prompt = g_prompt.replay
        import time
        t_pf = time.perf_counter()
        if batch_prefill:
            self._prefill_batch(list(prompt))  # logits of the last prompt token
        else:
            with torch.cuda.stream(self.stream):
                self._set_state(prompt[0], 0, fed=1)
                for _ in range(n_p - 1):
                    run_prompt()
                self._enqueue_layers()  # the last prompt token, with its logits
                self._enqueue_head()
            self.stream.synchronize()
        t_pf = time.perf_counter() - t_pf
        with torch.cuda.stream(self.stream):
            # the first token: argmax of the prompt's logits; state at the
            # last prompt position, prompt consumed
            self._set_state(0, n_p - 1, fed=0, count=0)
            if window is not None:
                window.copy_(torch.from_numpy(ring))
            advance()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(self.stream)
            left = n_gen - 1
            while run_gen_k is not None and left >= per_graph:
                run_gen_k()
                left -= per_graph
            for _ in range(left):
                run_gen()
            b.record(self.stream)
        self.stream.synchronize()
        if timing is not None:
            timing["gen_ms"] = a.elapsed_time(b)
            timing["steps"] = n_gen - 1
            timing["prefill_ms"] = t_pf * 1e3  # host wall clock, synchronized
        out = [int(t) for t in hist.cpu().tolist()]
        self.n_past = n_p + n_gen - 1
        self.cached_ids = list(prompt) + out[:-1]
        return out

    def _capture(self, fn):
        """One eager run of fn (sizes the library's per-stream workspace
        before capture), then a HIP graph of it on self.stream."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            fn()
        self.stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=self.stream):
            fn()
        self.stream.synchronize()
        return g


def synthetic_llama_1b(seed: int = 0, n_layer: int = 16, n_embd: int = 2048,
                       n_head: int = 32, n_kv: int = 8, n_ff: int = 8192,
                       n_vocab: int = 128256, n_ctx_train: int = 4096,
                       std: float = 0.02) -> tuple[Hyperparams, dict]:
    """The synthetic Llama-3.2-1B-shaped model of benchmark config 5: random
    zero-mean weights (synth.model_blocks), Q4_K everywhere except Q6_K for
    attn_v (all layers), ffn_down in the layers llama.cpp's Q4_K_M recipe
    gives more bits (i < n/8, i >= 7n/8, or (i - n/8) % 3 == 2: 8 of 16),
    and the untied output head; norm weights 1.0 (as make_bench_model.py
    writes them); RoPE theta 500000, eps 1e-5."""
    from . import synth
    head_dim = n_embd // n_head
    hp = Hyperparams(arch="llama", n_layer=n_layer, n_embd=n_embd, n_head=n_head,
                     n_kv=n_kv, n_ff=n_ff, n_vocab=n_vocab, n_ctx_train=n_ctx_train,
                     head_dim=head_dim, n_rot=head_dim, rms_eps=1e-5, rope_base=500000.0,
                     rope_style="norm")
    q_dim, kv_dim = n_head * head_dim, n_kv * head_dim
    tensors: dict = {}
    k = [0]

    def add(name, dtype, rows, cols):
        k[0] += 1
        tensors[name] = Tensor(dtype, (rows, cols),
                               synth.model_blocks(dtype, rows, cols, seed * 1000 + k[0], std).reshape(-1))

    ones = np.ones(n_embd, dtype=np.float32)
    add("token_embd.weight", "Q4_K", n_vocab, n_embd)
    for i in range(n_layer):
        p = f"blk.{i}."
        more_bits = (i < n_layer // 8 or i >= 7 * n_layer // 8
                     or (i - n_layer // 8) % 3 == 2)
        tensors[p + "attn_norm.weight"] = Tensor("F32", (n_embd,), ones)
        tensors[p + "ffn_norm.weight"] = Tensor("F32", (n_embd,), ones)
        add(p + "attn_q.weight", "Q4_K", q_dim, n_embd)
        add(p + "attn_k.weight", "Q4_K", kv_dim, n_embd)
        add(p + "attn_v.weight", "Q6_K", kv_dim, n_embd)
        add(p + "attn_output.weight", "Q4_K", n_embd, q_dim)
        add(p + "ffn_gate.weight", "Q4_K", n_ff, n_embd)
        add(p + "ffn_up.weight", "Q4_K", n_ff, n_embd)
        add(p + "ffn_down.weight", "Q6_K" if more_bits else "Q4_K", n_embd, n_ff)
    tensors["output_norm.weight"] = Tensor("F32", (n_embd,), ones)
    add("output.weight", "Q6_K", n_vocab, n_embd)
    return hp, tensors
