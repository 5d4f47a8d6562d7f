"""GPU: the C++ harness over the C ABI and the header-only C++ mirror
(voltattn_amd/host/voltattn.hpp), run as a child process.

``--selftest`` is the reference's own correctness gate (src/voltattn.cu:838-935:
7 formats x 6 shapes at G = 64, plus the quantized formats at G = 32);
``--selftest-ex`` drives the grouped-query, paged and append wrappers of the
mirror against the oracle's double reference, and checks the appended page
pool byte for byte against the oracle's quantizer."""
from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CLI = ROOT / "build" / "voltattn"

pytestmark = pytest.mark.gpu


def _run(mode: str) -> str:
    if not CLI.exists():
        pytest.fail(f"{CLI} is not built (python -m voltattn_amd.build)")
    print(f"cli {mode}", flush=True)
    r = subprocess.run([str(CLI), mode], capture_output=True, text=True, timeout=100)
    print(r.stdout[-4000:], r.stderr[-2000:], flush=True)
    assert r.returncode == 0, f"{mode} exit {r.returncode}:\n{r.stdout[-3000:]}\n{r.stderr[-2000:]}"
    return r.stdout


def test_cli_selftest():
    out = _run("--selftest")
    assert "all 72 cases passed" in out
    assert "FAIL" not in out


def test_cli_selftest_ex():
    out = _run("--selftest-ex")
    assert "all 42 grouped/paged cases passed" in out
    assert "FAIL" not in out and "MISMATCH" not in out
