"""GGUF block geometry of the quantized formats on the hot path.

dtype -> (block_elements, block_bytes, sub_block_len, affine), the table the
reference keeps in alpacca/quants.py:317-326 (QUANT_GEOMETRY).  The same
numbers are compiled into the C ABI (aq_geometry); tests check they agree.
"""
from __future__ import annotations

QK = 32      # elements per block of the classic formats
QK_K = 256   # elements per K-quant super-block

QUANT_GEOMETRY = {
    "Q8_0": (QK, 34, 32, False),
    "Q4_0": (QK, 18, 32, False),
    "Q4_1": (QK, 20, 32, True),
    "Q5_0": (QK, 22, 32, False),
    "Q5_1": (QK, 24, 32, True),
    "Q4_K": (QK_K, 144, 32, True),
    "Q5_K": (QK_K, 176, 32, True),
    "Q6_K": (QK_K, 210, 16, False),
}

__all__ = ["QK", "QK_K", "QUANT_GEOMETRY"]
