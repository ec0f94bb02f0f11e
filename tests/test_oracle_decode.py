"""Pins the decoding oracle (oracle/quants_ref.py) without importing the
reference: hand-derived known answers, three independent restatements that
must agree bit-for-bit, the bijection of the K-quant scale packing, and
planted mistakes that these checks must catch."""
from __future__ import annotations

import struct

import numpy as np
import pytest

from oracle import quants_ref as Q
from tests import smoke_patterns as SP


def f16(v: float) -> bytes:
    return struct.pack("<e", v)


# ------------------------------------------------------------ known answers --
# Each block below is written by hand and its expected values are worked out
# by hand from the bit layouts (reference alpacca/quants.py:50-224).

def kat_q8_0():
    qs = [0, 1, -1, 127, -128, 2] + [0] * 26
    blk = f16(0.5) + struct.pack("<32b", *qs)
    return blk, {0: 0.0, 1: 0.5, 2: -0.5, 3: 63.5, 4: -64.0, 5: 1.0}


def kat_q4_0():
    qs = bytearray(16)
    qs[0], qs[15] = 0x10, 0xF8
    return f16(2.0) + bytes(qs), {0: -16.0, 16: -14.0, 15: 0.0, 31: 14.0}


def kat_q4_1():
    qs = bytearray(16)
    qs[3] = 0x5A
    return f16(0.25) + f16(-1.0) + bytes(qs), {3: 1.5, 19: 0.25, 0: -1.0}


def kat_q5_0():
    qs = bytearray(16)
    qs[0], qs[1] = 0x30, 0x07
    blk = f16(1.0) + struct.pack("<I", 0x00010002) + bytes(qs)
    return blk, {0: -16.0, 1: 7.0, 16: 3.0, 17: -16.0}


def kat_q5_1():
    qs = bytearray(16)
    qs[15] = 0xF0
    blk = f16(0.5) + f16(0.25) + struct.pack("<I", 0x80000000) + bytes(qs)
    return blk, {31: 15.75, 15: 0.25}


KSCALES = bytes([0xC1, 2, 3, 4, 5, 6, 7, 8, 0x21, 0x43, 0x65, 0x87])
# sc = [1, 2, 3, 4, 49, 3, 5, 7], mn = [5, 6, 7, 8, 2, 4, 6, 8]
KQS = bytes(((l % 16) | ((15 - l % 16) << 4)) for l in range(128))


def kat_q4_k():
    blk = f16(1.0) + f16(0.5) + KSCALES + KQS
    return blk, {0: -2.5, 1: -1.5, 32: 27.0, 130: 97.0, 161: 40.0, 255: -4.0}


def kat_q5_k():
    qh = bytearray(32)
    qh[0] = 0b101
    blk = f16(1.0) + f16(0.5) + KSCALES + bytes(qh) + KQS
    return blk, {0: 13.5, 64: 44.5, 32: 27.0, 1: -1.5}


def kat_q6_k():
    ql = bytes(range(128))
    qh = bytearray(64)
    qh[0] = 0xE4
    sc = [1, -1, 2, -2, 3, -3, 4, -4, 5, -5, 6, -6, 7, -7, 8, -8]
    blk = ql + bytes(qh) + struct.pack("<16b", *sc) + f16(0.25)
    return blk, {0: -8.0, 32: -8.0, 64: 0.0, 96: 18.0, 17: 7.75, 200: -49.0}


KATS = {"Q8_0": kat_q8_0, "Q4_0": kat_q4_0, "Q4_1": kat_q4_1, "Q5_0": kat_q5_0,
        "Q5_1": kat_q5_1, "Q4_K": kat_q4_k, "Q5_K": kat_q5_k, "Q6_K": kat_q6_k}


def check_kat(dtype) -> bool:
    blk, want = KATS[dtype]()
    be = Q.GEOMETRY[dtype][0]
    assert len(blk) == Q.GEOMETRY[dtype][1]
    got = Q.dequantize(blk, be, dtype)
    return all(float(got[e]) == v for e, v in want.items())


@pytest.mark.parametrize("dtype", list(KATS))
def test_known_answers(dtype):
    assert check_kat(dtype)
    blk, want = KATS[dtype]()
    be = Q.GEOMETRY[dtype][0]
    for decoded in (Q.scalar_decode(blk, dtype), Q.exact_decode(blk, dtype)):
        assert all(float(decoded[e]) == v for e, v in want.items())


# ------------------------------------------------ three restatements agree --

def random_blocks(dtype, n, seed):
    """Uniform random bytes; fp16 fields finite, of both signs, spanning
    normal and subnormal magnitudes; K-quant scales over the full 0..255 and
    Q6_K int8 scales over the full -128..127 range."""
    be, bb, _, _ = Q.GEOMETRY[dtype]
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(n, bb), dtype=np.uint8)
    offs = {"Q6_K": [208], "Q4_K": [0, 2], "Q5_K": [0, 2], "Q4_1": [0, 2],
            "Q5_1": [0, 2]}.get(dtype, [0])
    for o in offs:
        mag = 10.0 ** rng.uniform(-7.5, 3.0, n)
        b[:, o:o + 2] = (mag * rng.choice([-1.0, 1.0], n)).astype("<f2").view(np.uint8).reshape(-1, 2)
    return b.tobytes()


@pytest.mark.parametrize("dtype", list(Q.GEOMETRY))
@pytest.mark.parametrize("seed", [0, 1])
def test_restatements_agree_bitwise(dtype, seed):
    be = Q.GEOMETRY[dtype][0]
    n_blocks = 6 if be == 256 else 40
    data = random_blocks(dtype, n_blocks, seed)
    vec = Q.dequantize(data, n_blocks * be, dtype)
    exact = Q.exact_decode(data, dtype)
    scal = Q.scalar_decode(data, dtype).astype(np.float32)
    assert np.array_equal(vec.view(np.uint32), exact.view(np.uint32))
    assert np.array_equal(vec, scal)


@pytest.mark.parametrize("fmt,rows,cols", SP.SMALL_CASES)
def test_reference_smoke_patterns_decode(fmt, rows, cols):
    """smoke.py:157-164: the NumPy decode agrees with the pure decoder; here
    all three restatements agree bit-for-bit on the reference's own blocks."""
    data = SP.packed(fmt, rows, cols, Q.quantize_q8_0, Q.quantize_q4_0)
    vec = Q.dequantize(data, rows * cols, fmt)
    assert np.array_equal(vec.view(np.uint32), Q.exact_decode(data, fmt).view(np.uint32))
    assert float(np.max(np.abs(vec - Q.scalar_decode(data, fmt)))) < 1e-6


@pytest.mark.parametrize("fmt,tol", [("Q8_0", 0.06), ("Q4_0", 0.6)])
def test_quantize_roundtrip(fmt, tol):
    """smoke.py:65-71 with the reference's own inputs and tolerances."""
    vals = [(i % 97) / 7.0 - 6.5 for i in range(512)]
    packed = Q.quantize_q8_0(vals) if fmt == "Q8_0" else Q.quantize_q4_0(vals)
    back = Q.dequantize(packed, len(vals), fmt)
    assert max(abs(a - b) for a, b in zip(vals, back)) < tol


def test_scale_packing_is_a_bijection():
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, size=(2000, 12), dtype=np.uint8)
    sc, mn = Q.kquant_scales(raw)
    assert sc.min() >= 0 and sc.max() <= 63 and mn.min() >= 0 and mn.max() <= 63
    for i in range(0, 2000, 97):
        assert Q.pack_kquant_scales(list(sc[i]), list(mn[i])) == bytes(raw[i])
    six = rng.integers(0, 64, size=(500, 16))
    for row in six:
        packed = np.frombuffer(Q.pack_kquant_scales(list(row[:8]), list(row[8:])), np.uint8)
        s2, m2 = Q.kquant_scales(packed[None, :])
        assert list(s2[0]) == list(row[:8]) and list(m2[0]) == list(row[8:])


def test_geometry_matches_product_table():
    from alpacca_amd.quants import QUANT_GEOMETRY
    assert QUANT_GEOMETRY == Q.GEOMETRY


# ---------------------------------------------------- planted mistakes ------

def test_planted_nibble_swap_is_caught(monkeypatch):
    monkeypatch.setattr(Q, "_K_NIB", 4 - Q._K_NIB)  # high/low nibble swapped
    assert not check_kat("Q4_K")


def test_planted_scale_index_is_caught(monkeypatch):
    def wrong(s):  # mins of sub-blocks 4..7 read s[j-4] instead of s[j]
        s = s.astype(np.int32)
        sc = np.concatenate([s[:, 0:4] & 63, (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)], 1)
        mn = np.concatenate([s[:, 4:8] & 63, (s[:, 8:12] >> 4) | ((s[:, 0:4] >> 6) << 4)], 1)
        return sc, mn
    monkeypatch.setattr(Q, "kquant_scales", wrong)
    assert not check_kat("Q4_K")


def test_planted_q6k_high_bits_are_caught(monkeypatch):
    monkeypatch.setattr(Q, "_Q6_QHSHIFT", Q._Q6_QHSHIFT[::-1].copy())
    assert not check_kat("Q6_K")


def test_planted_q5_bit_position_is_caught(monkeypatch):
    monkeypatch.setattr(Q, "_K_QHSHIFT", (Q._K_QHSHIFT + 1) % 8)
    assert not check_kat("Q5_K")


def test_planted_offset_is_caught(monkeypatch):
    real = Q._UNPACK["Q4_0"]

    def off_by_one(b):  # code = nibble - 7 instead of - 8
        q, d, m = real(b)
        return (q + 1).astype(np.int8), d, m
    monkeypatch.setitem(Q._UNPACK, "Q4_0", off_by_one)
    assert not check_kat("Q4_0")
