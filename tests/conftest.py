"""Shared pytest setup: repo root on sys.path and the `gpu` marker.

Tests marked `gpu` need a visible gfx950 device and the built HIP library
(alpacca_amd/_native/libalpacca_amd.so); everything else runs on the CPU.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an AMD gfx950 GPU and the built HIP library")
