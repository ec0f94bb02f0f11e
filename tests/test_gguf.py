"""GGUF reader/writer (alpacca_amd/gguf.py).

The reader is pinned by a file assembled by hand from the format's layout
(independent of our writer); the writer by round trips; the loader by the
reference's metadata keys (model.py:186-217) and, on the GPU, by greedy
tokens identical to the in-memory model's and the oracle's.
"""
from __future__ import annotations

import dataclasses
import struct

import numpy as np
import pytest

from alpacca_amd import gguf, synth
from alpacca_amd.model import synthetic_llama_1b


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _hand_file(tmp_path, alignment=None):
    """magic, v3, 2 tensors, kv: architecture, an int32 array, a float, a
    bool, (alignment); tensors: 'w' Q8_0 dims (64, 3) at 0, 'n' F32 (5,) after."""
    kv = [_s("general.architecture") + struct.pack("<I", 8) + _s("llama"),
          _s("x.ints") + struct.pack("<IIQ", 9, 5, 3) + struct.pack("<3i", -1, 2, 300),
          _s("x.eps") + struct.pack("<If", 6, 1e-5),
          _s("x.flag") + struct.pack("<IB", 7, 1)]
    if alignment:
        kv.append(_s("general.alignment") + struct.pack("<II", 4, alignment))
    align = alignment or 32
    w = np.random.default_rng(0).integers(0, 256, 3 * 2 * 34, dtype=np.uint8).tobytes()
    n = np.arange(5, dtype="<f4").tobytes()
    w_pad = (len(w) + align - 1) // align * align
    infos = (_s("w") + struct.pack("<I", 2) + struct.pack("<2Q", 64, 3) + struct.pack("<IQ", 8, 0)
             + _s("n") + struct.pack("<I", 1) + struct.pack("<Q", 5) + struct.pack("<IQ", 0, w_pad))
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, len(kv)) + b"".join(kv) + infos
    start = (len(head) + align - 1) // align * align
    blob = head + b"\0" * (start - len(head)) + w + b"\0" * (w_pad - len(w)) + n
    p = tmp_path / "hand.gguf"
    p.write_bytes(blob)
    return p, w, n, start


@pytest.mark.parametrize("alignment", [None, 64])
def test_reader_on_a_hand_assembled_file(tmp_path, alignment):
    p, w, n, start = _hand_file(tmp_path, alignment)
    with gguf.GGUFReader(p) as g:
        assert g.version == 3 and g.architecture == "llama"
        assert g.get("x.ints") == [-1, 2, 300]
        assert abs(g.get("x.eps") - 1e-5) < 1e-12 and g.get("x.flag") is True
        assert g.data_start == start and g.alignment == (alignment or 32)
        e = g.tensors["w"]
        assert (e.dims, e.dtype, e.offset, e.n_bytes) == ((64, 3), "Q8_0", 0, len(w))
        assert bytes(g.tensor_bytes("w")) == w
        assert bytes(g.tensor_bytes("n")) == n
        t = gguf.read_tensors(g)
        assert t["w"].shape == (3, 64) and bytes(t["w"].data) == w
        assert np.array_equal(t["n"].data, np.arange(5, dtype=np.float32))
        del t


def test_reader_rejects_bad_files(tmp_path):
    p, *_ = _hand_file(tmp_path)
    blob = p.read_bytes()
    for bad, msg in ((b"GGUX" + blob[4:], "not a GGUF"),
                     (blob[:4] + struct.pack("<I", 9) + blob[8:], "version"),
                     (blob[:40], "truncated"), (b"", "not a GGUF")):
        q = tmp_path / "bad.gguf"
        q.write_bytes(bad)
        with pytest.raises(ValueError, match=msg):
            gguf.GGUFReader(q)


@pytest.mark.parametrize("alignment", [32, 128])
def test_model_round_trip(tmp_path, alignment):
    hp, tensors = synthetic_llama_1b(seed=2, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=300, n_ctx_train=512)
    p = tmp_path / "m.gguf"
    gguf.write_model(p, hp, tensors, alignment=alignment)
    with gguf.GGUFReader(p) as g:
        # the format stores eps and the rope base as float32
        want = dataclasses.replace(hp, rms_eps=float(np.float32(hp.rms_eps)),
                                   rope_base=float(np.float32(hp.rope_base)))
        assert gguf.read_hyperparams(g) == want
        back = gguf.read_tensors(g)
        assert set(back) == set(tensors)
        for name, t in tensors.items():
            b = back[name]
            assert b.dtype == t.dtype and tuple(b.shape) == tuple(t.shape), name
            if t.dtype == "F32":
                assert np.array_equal(b.data, np.asarray(t.data, np.float32))
            else:
                assert bytes(b.data) == bytes(memoryview(t.data)), name
            assert g.tensors[name].offset % alignment == 0
        # the reference's keys (model.py:186-217)
        assert g.get("llama.attention.head_count_kv") == 2
        assert g.get("llama.rope.freq_base") == 500000.0
        del back


def test_hyperparams_defaults_and_errors(tmp_path):
    p = tmp_path / "x.gguf"
    gguf.write_gguf(p, [("general.architecture", gguf.T_STRING, "llama"),
                        ("llama.block_count", gguf.T_UINT32, 2),
                        ("llama.embedding_length", gguf.T_UINT32, 128),
                        ("llama.attention.head_count", gguf.T_UINT32, 2),
                        ("llama.feed_forward_length", gguf.T_UINT32, 256),
                        ("tokenizer.ggml.tokens", gguf.T_ARRAY,
                         (gguf.T_STRING, ["a", "b", "c"]))], [])
    with gguf.GGUFReader(p) as g:
        hp = gguf.read_hyperparams(g)
    # model.py:195-213 defaults: n_kv = n_head, head_dim = n_embd / n_head,
    # vocab from the token list, n_rot = head_dim, eps 1e-5, base 10000, ctx 4096
    assert (hp.n_kv, hp.head_dim, hp.n_vocab, hp.n_rot) == (2, 64, 3, 64)
    assert (hp.rms_eps, hp.rope_base, hp.n_ctx_train, hp.rope_style) == (1e-5, 10000.0, 4096, "norm")
    gguf.write_gguf(p, [("general.architecture", gguf.T_STRING, "gpt2")], [])
    with gguf.GGUFReader(p) as g, pytest.raises(ValueError, match="not supported"):
        gguf.read_hyperparams(g)
    with pytest.raises(ValueError, match="expected"):
        gguf.write_gguf(p, [], [("t", (256, 2), "Q4_K", b"\0" * 10)])


def test_writer_streams_ndarray_and_memoryview(tmp_path):
    blocks = synth.model_blocks("Q6_K", 4, 512, seed=1)
    p = tmp_path / "s.gguf"
    gguf.write_gguf(p, [], [("a", (512, 4), "Q6_K", blocks.reshape(-1)),
                            ("b", (512, 4), "Q6_K", memoryview(blocks.tobytes()))])
    with gguf.GGUFReader(p) as g:
        assert bytes(g.tensor_bytes("a")) == bytes(g.tensor_bytes("b")) == blocks.tobytes()


@pytest.mark.gpu
def test_load_model_greedy_matches(tmp_path):
    from alpacca_amd.model import Model
    from oracle.model_ref import RefModel
    hp, tensors = synthetic_llama_1b(seed=5, n_layer=2, n_embd=256, n_head=4, n_kv=2,
                                     n_ff=512, n_vocab=700, n_ctx_train=512)
    p = tmp_path / "m.gguf"
    gguf.write_model(p, hp, tensors)
    prompt = list(np.random.default_rng(3).integers(0, hp.n_vocab, 60))
    from_file = gguf.load_model(p).generate_greedy(prompt, 16)
    assert from_file == Model(hp, tensors).generate_greedy(prompt, 16)
    assert from_file == RefModel(hp, tensors).greedy(prompt, 16)[0]
