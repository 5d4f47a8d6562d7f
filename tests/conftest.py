"""pytest configuration: repo root on sys.path, the `gpu` marker, shared helpers.

Tests marked `gpu` need a gfx950 device and the built HIP library; they run on
the GPU box (`pytest -m gpu`). Everything else runs on the CPU (`-m "not gpu"`).
"""
import importlib.util
import os
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# One HIP runtime per process: the torch-binding tests share the process with
# the ctypes tests, so the library binds to PyTorch's runtime whichever of the
# two initialises the device first (voltattn_amd's VOLTATTN_HIP_RUNTIME).
if importlib.util.find_spec("torch") is not None:
    os.environ.setdefault("VOLTATTN_HIP_RUNTIME", "torch")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and libvoltattn_hip.so")
