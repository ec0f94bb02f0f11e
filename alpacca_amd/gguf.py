"""GGUF model files: the input side of the quantized path.

A reader (header, metadata key/values, tensor table, aligned data section,
zero-copy tensor bytes over an mmap) and a streaming writer, following the
GGUF v3 container layout (the ggml project's published file format, as the
reference's own alpacca/gguf.py:114-185 reads it and :199-301 writes it),
plus ``load_model``: the hyperparameters and tensors of a llama-family GGUF
turned into a device-resident ``alpacca_amd.model.Model`` - the part of the
reference's Model.load (alpacca/model.py:180-330) that touches the hot path.

Layout (all little-endian): magic "GGUF", u32 version (2 or 3), u64 tensor
count, u64 key/value count; key/values (string key, u32 value type, value);
tensor infos (string name, u32 n_dims, n_dims x u64 dims in ggml order -
dims[0] is the contiguous one -, u32 ggml type id, u64 offset into the data
section); padding to `general.alignment` (default 32); tensor data, each
tensor at its offset.  Strings are u64 length + UTF-8 bytes; arrays are u32
element type + u64 count + elements.
"""
from __future__ import annotations

import mmap
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

MAGIC = b"GGUF"
DEFAULT_ALIGNMENT = 32

# metadata value types
T_UINT8, T_INT8, T_UINT16, T_INT16 = 0, 1, 2, 3
T_UINT32, T_INT32, T_FLOAT32, T_BOOL = 4, 5, 6, 7
T_STRING, T_ARRAY, T_UINT64, T_INT64, T_FLOAT64 = 8, 9, 10, 11, 12
_SCALARS = {T_UINT8: "<u1", T_INT8: "<i1", T_UINT16: "<u2", T_INT16: "<i2",
            T_UINT32: "<u4", T_INT32: "<i4", T_FLOAT32: "<f4", T_UINT64: "<u8",
            T_INT64: "<i8", T_FLOAT64: "<f8", T_BOOL: "<u1"}

# ggml tensor type ids (gguf.py:36-43 of the reference names the same ids)
TYPE_IDS = {"F32": 0, "F16": 1, "Q4_0": 2, "Q4_1": 3, "Q5_0": 6, "Q5_1": 7, "Q8_0": 8,
            "Q8_1": 9, "Q2_K": 10, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14,
            "Q8_K": 15, "I8": 24, "I16": 25, "I32": 26, "I64": 27, "F64": 28, "BF16": 30}
TYPE_NAMES = {v: k for k, v in TYPE_IDS.items()}
# NumPy element types of the dense tensor types (BF16: the raw 16-bit words)
_DENSE_NP = {"F32": "<f4", "F16": "<f2", "BF16": "<u2"}
# (elements, bytes) per block
BLOCKS = {"F32": (1, 4), "F16": (1, 2), "BF16": (1, 2), "F64": (1, 8), "I8": (1, 1),
          "I16": (1, 2), "I32": (1, 4), "I64": (1, 8), "Q4_0": (32, 18), "Q4_1": (32, 20),
          "Q5_0": (32, 22), "Q5_1": (32, 24), "Q8_0": (32, 34), "Q8_1": (32, 36),
          "Q2_K": (256, 84), "Q3_K": (256, 110), "Q4_K": (256, 144), "Q5_K": (256, 176),
          "Q6_K": (256, 210), "Q8_K": (256, 292)}


@dataclass
class TensorEntry:
    name: str
    dims: tuple  # ggml order: dims[0] is contiguous
    dtype: str
    offset: int  # within the data section

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n

    @property
    def n_bytes(self) -> int:
        if self.dtype not in BLOCKS:
            raise ValueError(f"tensor {self.name}: unsupported type {self.dtype}")
        be, bb = BLOCKS[self.dtype]
        if self.n_elements % be:
            raise ValueError(f"tensor {self.name}: {self.n_elements} elements are not whole "
                             f"{self.dtype} blocks")
        return self.n_elements // be * bb


@dataclass
class GGUFReader:
    """A GGUF file opened read-only; tensor bytes are views of the mmap."""
    path: Path
    version: int = 0
    metadata: dict = field(default_factory=dict)
    tensors: dict = field(default_factory=dict)
    data_start: int = 0
    alignment: int = DEFAULT_ALIGNMENT

    def __post_init__(self):
        self.path = Path(self.path)
        self._fh = open(self.path, "rb")
        try:
            self._mm = mmap.mmap(self._fh.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:  # empty file
            self._fh.close()
            raise ValueError(f"{self.path} is not a GGUF file") from None
        try:
            self._parse()
        except Exception:
            self.close()
            raise

    def close(self) -> None:
        if getattr(self, "_mm", None) is not None:
            try:
                self._mm.close()
            except BufferError:  # tensor views still alive keep the map until
                pass             # they are released
            self._mm = None
        if getattr(self, "_fh", None) is not None:
            self._fh.close()
            self._fh = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    # -- parsing ---------------------------------------------------------

    def _parse(self) -> None:
        mm = self._mm
        if len(mm) < 24 or mm[:4] != MAGIC:
            raise ValueError(f"{self.path} is not a GGUF file")
        self.version, n_tensors, n_kv = struct.unpack_from("<IQQ", mm, 4)
        if self.version not in (2, 3):
            raise ValueError(f"unsupported GGUF version {self.version}")
        pos = 24

        def need(p, n):
            if p + n > len(mm):
                raise ValueError(f"{self.path}: truncated GGUF header")

        def string(p):
            need(p, 8)
            (n,) = struct.unpack_from("<Q", mm, p)
            need(p + 8, n)
            return bytes(mm[p + 8:p + 8 + n]).decode("utf-8", errors="replace"), p + 8 + n

        def value(t, p):
            if t in _SCALARS:
                dt = np.dtype(_SCALARS[t])
                need(p, dt.itemsize)
                v = np.frombuffer(mm, dtype=dt, count=1, offset=p)[0]
                v = bool(v) if t == T_BOOL else v.item()
                return v, p + dt.itemsize
            if t == T_STRING:
                return string(p)
            if t == T_ARRAY:
                need(p, 12)
                et, cnt = struct.unpack_from("<IQ", mm, p)
                p += 12
                if et in _SCALARS:  # one vectorized read
                    dt = np.dtype(_SCALARS[et])
                    need(p, cnt * dt.itemsize)
                    arr = np.frombuffer(mm, dtype=dt, count=cnt, offset=p)
                    vals = arr.astype(bool).tolist() if et == T_BOOL else arr.tolist()
                    return vals, p + cnt * dt.itemsize
                out = []
                for _ in range(cnt):
                    v, p = value(et, p)
                    out.append(v)
                return out, p
            raise ValueError(f"{self.path}: unknown metadata value type {t}")

        for _ in range(n_kv):
            key, pos = string(pos)
            need(pos, 4)
            (t,) = struct.unpack_from("<I", mm, pos)
            self.metadata[key], pos = value(t, pos + 4)
        for _ in range(n_tensors):
            name, pos = string(pos)
            need(pos, 4)
            (nd,) = struct.unpack_from("<I", mm, pos)
            need(pos + 4, 8 * nd + 12)
            dims = struct.unpack_from(f"<{nd}Q", mm, pos + 4)
            tid, off = struct.unpack_from("<IQ", mm, pos + 4 + 8 * nd)
            pos += 4 + 8 * nd + 12
            self.tensors[name] = TensorEntry(name, tuple(dims),
                                             TYPE_NAMES.get(tid, f"UNKNOWN_{tid}"), off)
        self.alignment = int(self.metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if self.alignment <= 0:
            raise ValueError(f"{self.path}: bad alignment {self.alignment}")
        self.data_start = (pos + self.alignment - 1) // self.alignment * self.alignment

    # -- access ----------------------------------------------------------

    def tensor_bytes(self, name: str) -> memoryview:
        """The tensor's raw bytes, zero-copy (a view of the mmap)."""
        if self._mm is None:
            raise ValueError(f"{self.path} is closed")
        e = self.tensors[name]
        start = self.data_start + e.offset
        end = start + e.n_bytes
        if end > len(self._mm):
            raise ValueError(f"tensor {name} runs past the end of {self.path}")
        return memoryview(self._mm)[start:end]

    def get(self, key: str, default: Any = None) -> Any:
        return self.metadata.get(key, default)

    @property
    def architecture(self) -> str:
        return str(self.metadata.get("general.architecture", ""))


# ---- writing ---------------------------------------------------------------

def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(t: int, v) -> bytes:
    if t == T_BOOL:
        return struct.pack("<B", 1 if v else 0)
    if t in _SCALARS:
        return np.array([v], dtype=_SCALARS[t]).tobytes()
    if t == T_STRING:
        return _pack_string(str(v))
    if t == T_ARRAY:
        et, vals = v
        head = struct.pack("<IQ", et, len(vals))
        if et in _SCALARS and et != T_BOOL:
            return head + np.asarray(vals, dtype=_SCALARS[et]).tobytes()
        return head + b"".join(_pack_value(et, x) for x in vals)
    raise ValueError(f"cannot write metadata type {t}")


def write_gguf(path, metadata: list, tensors: list, alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF v3 file.  metadata: [(key, type, value)] (arrays as
    (element type, values)); tensors: [(name, dims in ggml order, dtype,
    bytes-like)].  Tensor data is streamed (never concatenated in memory)."""
    kvs = list(metadata)
    if alignment != DEFAULT_ALIGNMENT and not any(k == "general.alignment" for k, _, _ in kvs):
        kvs.append(("general.alignment", T_UINT32, alignment))
    head = bytearray(MAGIC + struct.pack("<IQQ", 3, len(tensors), len(kvs)))
    for key, t, v in kvs:
        head += _pack_string(key) + struct.pack("<I", t) + _pack_value(t, v)
    offset, sizes = 0, []
    for name, dims, dtype, data in tensors:
        e = TensorEntry(name, tuple(int(d) for d in dims), dtype, offset)
        nbytes = memoryview(data).nbytes
        if nbytes != e.n_bytes:
            raise ValueError(f"{name}: {nbytes} bytes for {dtype} {tuple(dims)}, expected {e.n_bytes}")
        head += _pack_string(name) + struct.pack("<I", len(dims))
        head += struct.pack(f"<{len(dims)}Q", *e.dims) + struct.pack("<IQ", TYPE_IDS[dtype], offset)
        sizes.append(nbytes)
        offset += (nbytes + alignment - 1) // alignment * alignment
    data_start = (len(head) + alignment - 1) // alignment * alignment
    with open(path, "wb") as f:
        f.write(head)
        f.write(b"\0" * (data_start - len(head)))
        for (_, _, _, data), n in zip(tensors, sizes):
            f.write(memoryview(data).cast("B"))
            f.write(b"\0" * ((n + alignment - 1) // alignment * alignment - n))


# ---- models ------------------------------------------------------------------

def model_metadata(hp, n_vocab: int | None = None) -> list:
    """The metadata keys Model.load reads (alpacca/model.py:186-217) for hp."""
    a = hp.arch
    return [("general.architecture", T_STRING, a),
            (f"{a}.block_count", T_UINT32, hp.n_layer),
            (f"{a}.embedding_length", T_UINT32, hp.n_embd),
            (f"{a}.attention.head_count", T_UINT32, hp.n_head),
            (f"{a}.attention.head_count_kv", T_UINT32, hp.n_kv),
            (f"{a}.attention.key_length", T_UINT32, hp.head_dim),
            (f"{a}.feed_forward_length", T_UINT32, hp.n_ff),
            (f"{a}.vocab_size", T_UINT32, n_vocab or hp.n_vocab),
            (f"{a}.context_length", T_UINT32, hp.n_ctx_train),
            (f"{a}.rope.dimension_count", T_UINT32, hp.n_rot),
            (f"{a}.attention.layer_norm_rms_epsilon", T_FLOAT32, hp.rms_eps),
            (f"{a}.rope.freq_base", T_FLOAT32, hp.rope_base)]


def write_model(path, hp, tensors: dict, alignment: int = DEFAULT_ALIGNMENT) -> None:
    """A model given as (Hyperparams, {name: Tensor}) as a GGUF file: matrices
    (rows, cols) stored with ggml dims (cols, rows), vectors as F32."""
    out = []
    for name, t in tensors.items():
        if len(t.shape) == 1:
            v = np.ascontiguousarray(np.asarray(t.data, dtype="<f4").reshape(-1))
            out.append((name, (v.size,), "F32", v))
        else:
            rows, cols = t.shape
            data = t.data
            if t.dtype in _DENSE_NP and isinstance(data, np.ndarray) and data.dtype != np.uint8:
                data = np.ascontiguousarray(data, dtype=_DENSE_NP[t.dtype]).reshape(-1)
            out.append((name, (cols, rows), t.dtype, data))
    write_gguf(path, model_metadata(hp), out, alignment)


def read_hyperparams(g: GGUFReader):
    """Hyperparams from the metadata, as Model.load derives them
    (alpacca/model.py:186-217)."""
    from .model import ROPE_STYLES, Hyperparams
    arch = g.architecture
    if arch not in ROPE_STYLES:
        raise ValueError(f"architecture '{arch}' is not supported (supported: "
                         f"{', '.join(sorted(ROPE_STYLES))})")
    if int(g.get("split.count", 1) or 1) > 1:
        raise ValueError("multi-part (split) GGUFs are not supported")

    def meta(key, default=None):
        return g.get(f"{arch}.{key}", default)

    n_embd = int(meta("embedding_length"))
    n_head = int(meta("attention.head_count"))
    n_kv = int(meta("attention.head_count_kv", n_head) or n_head)
    head_dim = int(meta("attention.key_length", n_embd // n_head) or n_embd // n_head)
    return Hyperparams(
        arch=arch, n_layer=int(meta("block_count")), n_embd=n_embd, n_head=n_head, n_kv=n_kv,
        n_ff=int(meta("feed_forward_length")),
        n_vocab=int(g.get(f"{arch}.vocab_size", len(g.get("tokenizer.ggml.tokens", [])))),
        n_ctx_train=int(meta("context_length", 4096)), head_dim=head_dim,
        n_rot=int(meta("rope.dimension_count", head_dim) or head_dim),
        rms_eps=float(meta("attention.layer_norm_rms_epsilon", 1e-5)),
        rope_base=float(meta("rope.freq_base", 10000.0)), rope_style=ROPE_STYLES[arch])


def _dense_values(raw, dtype: str) -> np.ndarray:
    """F32 / F16 / BF16 bytes as float32 values (quants.py:517-523)."""
    if dtype == "BF16":
        return (np.frombuffer(raw, dtype="<u2").astype(np.uint32) << 16).view(np.float32)
    return np.frombuffer(raw, dtype=_DENSE_NP[dtype]).astype(np.float32)


def read_tensors(g: GGUFReader) -> dict:
    """{name: Tensor}: 2-D tensors as (rows, cols) = (dims[1], dims[0]) with
    their raw bytes (mmap views; F32/F16/BF16 matrices keep their stored
    type and become dense matrices); 1-D F32/F16/BF16 tensors as float32
    arrays."""
    from .model import Tensor
    out = {}
    for name, e in g.tensors.items():
        raw = g.tensor_bytes(name)
        if len(e.dims) == 1:
            if e.dtype not in _DENSE_NP:
                raise ValueError(f"tensor {name}: {e.dtype} vectors are not supported")
            out[name] = Tensor("F32", (e.n_elements,), _dense_values(raw, e.dtype))
        else:
            out[name] = Tensor(e.dtype, (int(np.prod(e.dims[1:])), e.dims[0]), raw)
    return out


def load_model(path, n_ctx: int = 0, **kw):
    """Model.load for the device path: a llama-family GGUF with quantized
    (or F32/F16/BF16 dense) matrices becomes an alpacca_amd.model.Model
    (weights uploaded to HBM once; the file is closed afterwards, as
    model.py:340-341 does)."""
    from .model import Model
    with GGUFReader(path) as g:
        hp = read_hyperparams(g)
        tensors = read_tensors(g)
        m = Model(hp, tensors, n_ctx=n_ctx, **kw)
        del tensors
    return m
