"""Oracle: GGUF block decoders (TEST INFRASTRUCTURE - see oracle/__init__.py).

Three independent restatements of the reference's decoding
(jtiro232/Alpacca alpacca/quants.py):

1. ``unpack`` / ``dequantize``: vectorized NumPy, built on per-element index
   tables, giving (codes int8, d_eff f32, m_eff f32|None) and the float32
   values ``f32(code) * d_eff (+ m_eff)`` exactly as the reference assembles
   them (quants.py:338-504 unpackers, :498-504 _np_assemble, :507-528
   dequantize).
2. ``scalar_decode``: one block at a time in Python floats, following the
   loop structure of the reference's pure decoders (quants.py:50-224).
3. ``exact_decode``: the exact rational value of every element
   (fractions.Fraction) rounded once to float32 (round-to-nearest-even).

The tests require (1) == RN_f32(3) bit-for-bit (the reference's float32 value
is exact up to that single rounding, because every scale product fits in 24
bits) and (1) == f32((2)).
"""
from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np

QK = 32
QK_K = 256

# quants.py:317-326
GEOMETRY = {
    "Q8_0": (QK, 34, 32, False),
    "Q4_0": (QK, 18, 32, False),
    "Q4_1": (QK, 20, 32, True),
    "Q5_0": (QK, 22, 32, False),
    "Q5_1": (QK, 24, 32, True),
    "Q4_K": (QK_K, 144, 32, True),
    "Q5_K": (QK_K, 176, 32, True),
    "Q6_K": (QK_K, 210, 16, False),
}


# ---------------------------------------------------------------- helpers ---

def block_view(data, dtype: str) -> np.ndarray:
    """Raw bytes as (n_blocks, block_bytes) uint8."""
    bb = GEOMETRY[dtype][1]
    arr = np.frombuffer(data, dtype=np.uint8)
    if arr.size % bb:
        raise ValueError(f"{dtype}: {arr.size} bytes is not a whole number of blocks")
    return arr.reshape(-1, bb)


def f16_field(b: np.ndarray, off: int) -> np.ndarray:
    """Little-endian fp16 at byte `off` of every block -> float32 (exact)."""
    return np.ascontiguousarray(b[:, off:off + 2]).view("<f2").reshape(-1).astype(np.float32)


def kquant_scales(s: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """12 packed bytes -> 8 six-bit scales and 8 six-bit mins (quants.py:127-133)."""
    s = s.astype(np.int32)
    lo_sc, lo_mn = s[:, 0:4] & 63, s[:, 4:8] & 63
    hi_sc = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    hi_mn = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return np.concatenate([lo_sc, hi_sc], 1), np.concatenate([lo_mn, hi_mn], 1)


def pack_kquant_scales(sc, mn) -> bytes:
    """Inverse of kquant_scales for one block: 8 scales + 8 mins (0..63)."""
    s = [0] * 12
    for j in range(4):
        s[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        s[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        s[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return bytes(s)


# element-order index tables ------------------------------------------------
# Q4_K / Q5_K: element e = 64c + 32h + l  <-  qs[32c + l], nibble h
_E = np.arange(256)
_K_QS = 32 * (_E // 64) + (_E % 32)
_K_NIB = 4 * ((_E // 32) % 2)
_K_QHSHIFT = (_E // 32)            # bit (2c + h) of qh[l]
_K_QHIDX = _E % 32
# Q6_K: element e = 128hf + 32g + l
_HF, _G, _L = _E // 128, (_E % 128) // 32, _E % 32
_Q6_QL = 64 * _HF + 32 * (_G & 1) + _L
_Q6_NIB = 4 * (_G >> 1)
_Q6_QH = 32 * _HF + _L
_Q6_QHSHIFT = 2 * _G
# classic 32-element formats: element e < 16 low nibble of qs[e], else high of qs[e-16]
_C_QS = np.arange(32) % 16
_C_NIB = 4 * (np.arange(32) // 16)
# shift amounts as uint8, so that shifting the uint8 payload stays uint8 (int64
# shift tables would widen every byte to 64 bits; same values either way)
_K_NIB, _K_QHSHIFT, _Q6_NIB, _Q6_QHSHIFT, _C_NIB = (
    a.astype(np.uint8) for a in (_K_NIB, _K_QHSHIFT, _Q6_NIB, _Q6_QHSHIFT, _C_NIB))


def _unpack_q8_0(b):
    d = f16_field(b, 0)
    return b[:, 2:34].copy().view(np.int8), d[:, None], None


def _nibbles32(qs):
    return (qs[:, _C_QS] >> _C_NIB) & 15


def _qh_bits32(b, off):
    qh = np.ascontiguousarray(b[:, off:off + 4]).view("<u4").reshape(-1, 1)
    return ((qh >> np.arange(32, dtype=np.uint32)) & 1).astype(np.uint8)


def _unpack_q4_0(b):
    q = _nibbles32(b[:, 2:18]).astype(np.int16) - 8
    return q.astype(np.int8), f16_field(b, 0)[:, None], None


def _unpack_q4_1(b):
    q = _nibbles32(b[:, 4:20]).astype(np.int8)
    return q, f16_field(b, 0)[:, None], f16_field(b, 2)[:, None]


def _unpack_q5_0(b):
    q = (_nibbles32(b[:, 6:22]) | (_qh_bits32(b, 2) << 4)).astype(np.int16) - 16
    return q.astype(np.int8), f16_field(b, 0)[:, None], None


def _unpack_q5_1(b):
    q = (_nibbles32(b[:, 8:24]) | (_qh_bits32(b, 4) << 4)).astype(np.int8)
    return q, f16_field(b, 0)[:, None], f16_field(b, 2)[:, None]


def _kquant_scale_pair(b):
    d, dmin = f16_field(b, 0), f16_field(b, 2)
    sc, mn = kquant_scales(b[:, 4:16])
    return d[:, None] * sc.astype(np.float32), -(dmin[:, None] * mn.astype(np.float32))


def _unpack_q4_k(b):
    qs = b[:, 16:144]
    q = ((qs[:, _K_QS] >> _K_NIB) & 15).astype(np.int8)
    d_eff, m_eff = _kquant_scale_pair(b)
    return q, d_eff, m_eff


def _unpack_q5_k(b):
    qs, qh = b[:, 48:176], b[:, 16:48]
    hi = (qh[:, _K_QHIDX] >> _K_QHSHIFT) & 1
    q = (((qs[:, _K_QS] >> _K_NIB) & 15) | (hi << 4)).astype(np.int8)
    d_eff, m_eff = _kquant_scale_pair(b)
    return q, d_eff, m_eff


def _unpack_q6_k(b):
    ql, qh = b[:, 0:128], b[:, 128:192]
    q = (((ql[:, _Q6_QL] >> _Q6_NIB) & 15) |
         (((qh[:, _Q6_QH] >> _Q6_QHSHIFT) & 3) << 4)).astype(np.int16) - 32
    sc = b[:, 192:208].copy().view(np.int8).astype(np.float32)
    return q.astype(np.int8), f16_field(b, 208)[:, None] * sc, None


_UNPACK = {"Q8_0": _unpack_q8_0, "Q4_0": _unpack_q4_0, "Q4_1": _unpack_q4_1,
           "Q5_0": _unpack_q5_0, "Q5_1": _unpack_q5_1, "Q4_K": _unpack_q4_k,
           "Q5_K": _unpack_q5_k, "Q6_K": _unpack_q6_k}


def unpack(data, n: int, dtype: str):
    """Raw blocks of n elements -> (codes int8 (nb, block), d_eff f32 (nb, n_sub),
    m_eff f32 (nb, n_sub) | None).  Restates quants.np_unpack (quants.py:481-495)."""
    be = GEOMETRY[dtype][0]
    if n % be:
        raise ValueError(f"{dtype} needs a multiple of {be} elements")
    b = block_view(data, dtype)
    if b.shape[0] != n // be:
        raise ValueError(f"{dtype}: {b.shape[0]} blocks for {n} elements")
    q, d, m = _UNPACK[dtype](b)
    n_sub = be // GEOMETRY[dtype][2]
    d = np.broadcast_to(d, (b.shape[0], n_sub)).astype(np.float32)
    if m is not None:
        m = np.broadcast_to(m, (b.shape[0], n_sub)).astype(np.float32)
    return np.ascontiguousarray(q), np.ascontiguousarray(d), (
        None if m is None else np.ascontiguousarray(m))


def assemble(q, d_eff, m_eff, sub_len):
    """f32(code) * d_eff (+ m_eff), float32 (quants.py:498-504)."""
    nb, be = q.shape
    out = q.astype(np.float32).reshape(nb, be // sub_len, sub_len)
    out *= d_eff[:, :, None]
    if m_eff is not None:
        out += m_eff[:, :, None]
    return out.reshape(-1)


DENSE_WIDTH = {"F32": 4, "F16": 2, "BF16": 2}


def dense_decode(data, n: int, dtype: str) -> np.ndarray:
    """F32 / F16 / BF16 values to float32, exactly (quants.py:517-523):
    F32 as is, F16 by IEEE half -> single, BF16 as the upper 16 bits of a
    single."""
    raw = np.frombuffer(data, dtype=np.uint8)
    if raw.size != n * DENSE_WIDTH[dtype]:
        raise ValueError("wrong byte length")
    if dtype == "F32":
        return raw.view("<f4").astype(np.float32)
    if dtype == "F16":
        return raw.view("<f2").astype(np.float32)
    return (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)


def dequantize(data, n: int, dtype: str) -> np.ndarray:
    """Decode n elements to float32 (quants.py:507-528, NumPy branch)."""
    if dtype in DENSE_WIDTH:
        return dense_decode(data, n, dtype)
    q, d, m = unpack(data, n, dtype)
    return assemble(q, d, m, GEOMETRY[dtype][2])


# ------------------------------------------------------ scalar restatement --

def _f16s(raw, off):
    return struct.unpack_from("<e", raw, off)[0]


def _scalar_kscale(j, s):
    if j < 4:
        return s[j] & 63, s[j + 4] & 63
    return ((s[j + 4] & 15) | ((s[j - 4] >> 6) << 4),
            (s[j + 4] >> 4) | ((s[j] >> 6) << 4))


def _scalar_block(raw: bytes, dtype: str) -> list[float]:
    out = []
    if dtype == "Q8_0":
        d = _f16s(raw, 0)
        out = [d * v for v in struct.unpack_from("<32b", raw, 2)]
    elif dtype in ("Q4_0", "Q4_1", "Q5_0", "Q5_1"):
        d = _f16s(raw, 0)
        m = _f16s(raw, 2) if dtype in ("Q4_1", "Q5_1") else 0.0
        qh = 0
        if dtype == "Q5_0":
            qh = struct.unpack_from("<I", raw, 2)[0]
        elif dtype == "Q5_1":
            qh = struct.unpack_from("<I", raw, 4)[0]
        qs_off = {"Q4_0": 2, "Q4_1": 4, "Q5_0": 6, "Q5_1": 8}[dtype]
        bias = {"Q4_0": 8, "Q4_1": 0, "Q5_0": 16, "Q5_1": 0}[dtype]
        lo, hi = [0.0] * 16, [0.0] * 16
        for j in range(16):
            byte = raw[qs_off + j]
            a, b = byte & 15, byte >> 4
            if dtype in ("Q5_0", "Q5_1"):
                a |= ((qh >> j) & 1) << 4
                b |= ((qh >> (j + 16)) & 1) << 4
            lo[j] = d * (a - bias) + m
            hi[j] = d * (b - bias) + m
        out = lo + hi
    elif dtype in ("Q4_K", "Q5_K"):
        d, dmin = _f16s(raw, 0), _f16s(raw, 2)
        s = raw[4:16]
        qs = raw[48:176] if dtype == "Q5_K" else raw[16:144]
        qh = raw[16:48] if dtype == "Q5_K" else None
        for c in range(4):
            for h in range(2):
                sc, mn = _scalar_kscale(2 * c + h, s)
                for l in range(32):
                    v = (qs[32 * c + l] >> (4 * h)) & 15
                    if qh is not None:
                        v += 16 * ((qh[l] >> (2 * c + h)) & 1)
                    out.append(d * sc * v - dmin * mn)
    elif dtype == "Q6_K":
        ql, qh = raw[0:128], raw[128:192]
        sc = struct.unpack_from("<16b", raw, 192)
        d = _f16s(raw, 208)
        vals = [0.0] * 256
        for hf in range(2):
            for l in range(32):
                L, H = ql[64 * hf:], qh[32 * hf:]
                q = ((L[l] & 15) | ((H[l] & 3) << 4),
                     (L[32 + l] & 15) | (((H[l] >> 2) & 3) << 4),
                     (L[l] >> 4) | (((H[l] >> 4) & 3) << 4),
                     (L[32 + l] >> 4) | (((H[l] >> 6) & 3) << 4))
                for g in range(4):
                    e = 128 * hf + 32 * g + l
                    vals[e] = d * sc[e // 16] * (q[g] - 32)
        out = vals
    else:
        raise ValueError(dtype)
    return out


def scalar_decode(data, dtype: str) -> np.ndarray:
    """Block-by-block Python-float decode (quants.py:50-224), float64 values."""
    bb = GEOMETRY[dtype][1]
    raw = bytes(data)
    vals: list[float] = []
    for off in range(0, len(raw), bb):
        vals.extend(_scalar_block(raw[off:off + bb], dtype))
    return np.asarray(vals, dtype=np.float64)


# ------------------------------------------------------- exact rationals ---

def _round_f32(x: Fraction) -> np.float32:
    """Round an exact rational to the nearest float32 (ties to even)."""
    if x == 0:
        return np.float32(0.0)
    guess = np.float32(float(x))
    cands = {guess, np.nextafter(guess, np.float32(np.inf)),
             np.nextafter(guess, np.float32(-np.inf))}
    best = None
    for c in cands:
        if not np.isfinite(c):
            continue
        err = abs(Fraction(float(c)) - x)
        key = (err, int(np.float32(c).view(np.uint32)) & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return np.float32(best[1])


def element_code(raw: bytes, dtype: str, e: int) -> int:
    """Code of element e of one block, straight from the per-element bit
    layout (quants.py:50-224 read as closed forms), independent of both the
    index tables of `unpack` and the loops of `scalar_decode`."""
    if dtype == "Q8_0":
        return struct.unpack_from("<b", raw, 2 + e)[0]
    if dtype in ("Q4_0", "Q4_1", "Q5_0", "Q5_1"):
        qs_off = {"Q4_0": 2, "Q4_1": 4, "Q5_0": 6, "Q5_1": 8}[dtype]
        nib = (raw[qs_off + e % 16] >> (4 * (e // 16))) & 15
        if dtype in ("Q5_0", "Q5_1"):
            qh = struct.unpack_from("<I", raw, 2 if dtype == "Q5_0" else 4)[0]
            nib += 16 * ((qh >> e) & 1)
        return nib - {"Q4_0": 8, "Q5_0": 16}.get(dtype, 0)
    if dtype in ("Q4_K", "Q5_K"):
        c, h, l = e // 64, (e // 32) % 2, e % 32
        qs_off = 48 if dtype == "Q5_K" else 16
        v = (raw[qs_off + 32 * c + l] >> (4 * h)) & 15
        if dtype == "Q5_K":
            v += 16 * ((raw[16 + l] >> (2 * c + h)) & 1)
        return v
    if dtype == "Q6_K":
        hf, g, l = e // 128, (e % 128) // 32, e % 32
        low = (raw[64 * hf + 32 * (g % 2) + l] >> (4 * (g // 2))) & 15
        high = (raw[128 + 32 * hf + l] >> (2 * g)) & 3
        return low + 16 * high - 32
    raise ValueError(dtype)


def exact_decode(data, dtype: str) -> np.ndarray:
    """Exact value of every element, rounded once to float32: codes from
    `element_code`, fp16 fields decoded by struct, K-quant scales from the
    packing of quants.py:127-133, all arithmetic in fractions.Fraction."""
    be, bb, sub, _aff = GEOMETRY[dtype]
    raw_all = bytes(data)
    n_blocks = len(raw_all) // bb
    out = np.empty(n_blocks * be, dtype=np.float32)
    for i in range(n_blocks):
        raw = raw_all[i * bb:(i + 1) * bb]
        if dtype in ("Q4_K", "Q5_K"):
            d, dmin = Fraction(_f16s(raw, 0)), Fraction(_f16s(raw, 2))
            pairs = [_scalar_kscale(k, raw[4:16]) for k in range(8)]
            deff = [d * sc for sc, _ in pairs]
            meff = [-dmin * mn for _, mn in pairs]
            df, dmf = np.float32(_f16s(raw, 0)), np.float32(_f16s(raw, 2))
            deff_f = [df * np.float32(sc) for sc, _ in pairs]
            meff_f = [-(dmf * np.float32(mn)) for _, mn in pairs]
        elif dtype == "Q6_K":
            d = Fraction(_f16s(raw, 208))
            scs = struct.unpack_from("<16b", raw, 192)
            deff = [d * s for s in scs]
            meff = [Fraction(0)] * 16
            deff_f = [np.float32(_f16s(raw, 208)) * np.float32(s) for s in scs]
            meff_f = []
        else:
            d = Fraction(_f16s(raw, 0))
            m = Fraction(_f16s(raw, 2)) if dtype in ("Q4_1", "Q5_1") else Fraction(0)
            deff, meff = [d], [m]
            deff_f = [np.float32(_f16s(raw, 0))]
            meff_f = [np.float32(_f16s(raw, 2))] if dtype in ("Q4_1", "Q5_1") else []
        for e in range(be):
            s = e // sub
            code = element_code(raw, dtype, e)
            x = code * deff[s] + meff[s]
            if x == 0:
                # an exact zero: every operation was exact, so float32 IEEE
                # arithmetic on the same operands gives its sign (-0.0 when
                # a zero code meets a negative scale, as in the reference)
                out[i * be + e] = (np.float32(code) * np.float32(deff_f[s])
                                   + np.float32(meff_f[s])) if meff_f else (
                    np.float32(code) * np.float32(deff_f[s]))
            else:
                out[i * be + e] = _round_f32(x)
    return out


# ------------------------------------------------------------- encoders ----

def quantize_q8_0(values) -> bytes:
    """Restates quants.quantize_q8_0 (quants.py:533-544)."""
    if len(values) % QK:
        raise ValueError("Q8_0 needs a multiple of 32 values")
    out = bytearray()
    for i in range(0, len(values), QK):
        blk = values[i:i + QK]
        amax = max(abs(v) for v in blk)
        d = amax / 127.0 if amax else 0.0
        inv = 1.0 / d if d else 0.0
        out += struct.pack("<e32b", d, *[max(-128, min(127, round(v * inv))) for v in blk])
    return bytes(out)


def quantize_q4_0(values) -> bytes:
    """Restates quants.quantize_q4_0 (quants.py:547-559)."""
    if len(values) % QK:
        raise ValueError("Q4_0 needs a multiple of 32 values")
    out = bytearray()
    for i in range(0, len(values), QK):
        blk = values[i:i + QK]
        vmax = max(blk, key=abs)
        d = vmax / -8.0
        inv = 1.0 / d if d else 0.0
        q = [max(0, min(15, int(v * inv + 8.5))) for v in blk]
        out += struct.pack("<e", d) + bytes((q[j] & 15) | (q[j + 16] << 4) for j in range(16))
    return bytes(out)
