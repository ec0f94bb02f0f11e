"""The reference's own deterministic test inputs (tests/smoke.py:75-137):
closed-form byte patterns for Q4_K/Q5_K/Q6_K/Q4_1/Q5_0/Q5_1 blocks, the
weight/activation formulas, and the reference's tolerances for them.  These
are data generators (formulas of the reference's fixtures), used by both the
oracle tests and the GPU parity tests."""
from __future__ import annotations

import struct


def q4_k_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 256):
        d = 0.015625 + (blk % 7) * 0.001953125
        dmin = 0.00390625 + (blk % 5) * 0.0009765625
        out += struct.pack("<ee", d, dmin)
        out += bytes(((blk * 17 + i * 29) & 0xFF) for i in range(12))
        out += bytes(((blk * 31 + i * 7) & 0xFF) for i in range(128))
    return bytes(out)


def q5_k_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 256):
        d = 0.015625 + (blk % 7) * 0.001953125
        dmin = 0.00390625 + (blk % 5) * 0.0009765625
        out += struct.pack("<ee", d, dmin)
        out += bytes(((blk * 17 + i * 29) & 0xFF) for i in range(12))
        out += bytes(((blk * 23 + i * 13) & 0xFF) for i in range(32))
        out += bytes(((blk * 31 + i * 7) & 0xFF) for i in range(128))
    return bytes(out)


def q6_k_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 256):
        out += bytes(((blk * 13 + i * 11) & 0xFF) for i in range(128))
        out += bytes(((blk * 19 + i * 5) & 0xFF) for i in range(64))
        out += struct.pack("<16b", *[((blk * 7 + i * 9) % 63) - 31 for i in range(16)])
        out += struct.pack("<e", 0.001953125 + (blk % 5) * 0.000244140625)
    return bytes(out)


def q4_1_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 32):
        out += struct.pack("<ee", 0.015625 + (blk % 7) * 0.001953125,
                           -0.125 + (blk % 5) * 0.0625)
        out += bytes(((blk * 31 + i * 7) & 0xFF) for i in range(16))
    return bytes(out)


def q5_0_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 32):
        out += struct.pack("<e", 0.015625 + (blk % 7) * 0.001953125)
        out += bytes(((blk * 23 + i * 13) & 0xFF) for i in range(4))
        out += bytes(((blk * 31 + i * 7) & 0xFF) for i in range(16))
    return bytes(out)


def q5_1_bytes(n: int) -> bytes:
    out = bytearray()
    for blk in range(n // 32):
        out += struct.pack("<ee", 0.015625 + (blk % 7) * 0.001953125,
                           -0.125 + (blk % 5) * 0.0625)
        out += bytes(((blk * 23 + i * 13) & 0xFF) for i in range(4))
        out += bytes(((blk * 31 + i * 7) & 0xFF) for i in range(16))
    return bytes(out)


def weights(n: int) -> list[float]:
    return [((i * 37) % 251) / 17.0 - 7.0 for i in range(n)]


def x_vector(cols: int) -> list[float]:
    return [((i * 19) % 67) / 23.0 - 1.4 for i in range(cols)]


def packed(fmt: str, rows: int, cols: int, quantize_q8_0, quantize_q4_0) -> bytes:
    """The matrix bytes smoke.py's check_quantized_matvec builds (:134-155)."""
    n = rows * cols
    if fmt == "Q8_0":
        return quantize_q8_0(weights(n))
    if fmt == "Q4_0":
        return quantize_q4_0(weights(n))
    return {"Q4_1": q4_1_bytes, "Q5_0": q5_0_bytes, "Q5_1": q5_1_bytes,
            "Q4_K": q4_k_bytes, "Q5_K": q5_k_bytes, "Q6_K": q6_k_bytes}[fmt](n)


# (format, rows, cols) of smoke.py:310-317 and the large-matrix branch :318-358
SMALL_CASES = [("Q8_0", 5, 64), ("Q4_0", 5, 64), ("Q4_1", 5, 64), ("Q5_0", 5, 64),
               ("Q5_1", 5, 64), ("Q4_K", 3, 512), ("Q5_K", 3, 512), ("Q6_K", 3, 512)]
LARGE_CASES = [("Q4_K", 2112, 512), ("Q6_K", 2112, 512)]
