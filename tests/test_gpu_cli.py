"""GPU: the C++ harness over the C ABI and the header-only C++ mirror
(voltattn_amd/host/voltattn.hpp), run as a child process.

``--selftest`` is the reference's own correctness gate (src/voltattn.cu:838-935:
7 formats x 6 shapes at G = 64, plus the quantized formats at G = 32);
``--selftest-ex`` drives the grouped-query, paged and append wrappers of the
mirror against the oracle's double reference, and checks the appended page
pool byte for byte against the oracle's quantizer. ``--bench`` (gated on the
selftest, src/voltattn.cu:1075-1076) and ``--probe`` run on a small row set:
the table and its JSON copy carry every row with consistent figures."""
from __future__ import annotations

import json
import subprocess
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
CLI = ROOT / "build" / "voltattn"

pytestmark = pytest.mark.gpu


def _run(mode: str, *args: str, timeout: int = 100) -> str:
    if not CLI.exists():
        pytest.fail(f"{CLI} is not built (python -m voltattn_amd.build)")
    print(f"cli {mode} {' '.join(args)}", flush=True)
    r = subprocess.run([str(CLI), mode, *args], capture_output=True, text=True, timeout=timeout)
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


def test_cli_probe():
    out = _run("--probe")
    gbs = float(out.split("measured read ceiling:")[1].split("GB/s")[0])
    assert 1000.0 < gbs < 20000.0, gbs


def test_cli_bench_rows_and_json():
    with tempfile.TemporaryDirectory() as d:
        js = Path(d) / "bench.json"
        out = _run("--bench", "--L", "4096", "--fmt", "q8,q8+,q4+", "--reps", "5", "--set-gib", "0.5",
                   "--no-cpu", "--json", str(js), timeout=200)
        assert "all 72 cases passed" in out                  # the bench's selftest gate
        rows = json.loads(js.read_text())
    table = [ln for ln in out.splitlines() if ln.startswith("| q")]
    assert [ln.split("|")[1].strip() for ln in table] == ["q8", "q8+", "q4+"], table
    assert 1000.0 < rows["ceiling_gbps"] < 20000.0 and rows["G"] == 32
    assert [r["fmt"] for r in rows["rows"]] == ["q8", "q8+", "q4+"]
    for r in rows["rows"]:
        assert r["L"] == 4096 and r["S"] >= 1 and r["copies"] >= 1
        assert 0.0 < r["best_ms"] and 0.0 < r["mean_ms"] < 1.0, r
        assert abs(r["gbps"] - r["bytes"] / (r["best_ms"] * 1e6)) <= 1e-6 * r["gbps"], r
        assert 0.0 < r["mbu"] < 1.5, r
    # payload + scales of q8 and q4 at H=32, D=128, L=4096, G=32 (2*H*L*(D*b/8 + 2*D/G))
    assert [r["bytes"] for r in rows["rows"]] == [2 * 32 * 4096 * (128 + 8)] * 2 + [2 * 32 * 4096 * (64 + 8)]
