"""Pytest setup: the `gpu` marker and the repository root on sys.path.

Tests marked `gpu` need a ROCm device and the built `libhummingbird_amd.so`; everything else runs on the CPU.
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU and the built HIP library")
