"""pytest configuration: repo root on sys.path, the `gpu` marker, shared helpers.

Tests marked `gpu` need a gfx950 device and the built HIP library; they run on
the GPU box (`pytest -m gpu`). Everything else runs on the CPU (`-m "not gpu"`).
"""
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and libvoltattn_hip.so")
