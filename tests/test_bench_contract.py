"""bench.py's driver contract.

CPU: more than one GPU is refused with a message and no JSON line (this build
measures one MI355X). GPU: a short run prints exactly one JSON line on stdout
carrying every field the driver and the roofline/cpu_baseline contract name,
with consistent values (value = 1000 / ms_per_step, frac = achieved / peak,
the output check passed)."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
BENCH = ROOT / "bench.py"


@pytest.mark.parametrize("n", [2, 8])
def test_more_than_one_gpu_is_refused(n):
    r = subprocess.run([sys.executable, str(BENCH), "--gpus", str(n), "--steps", "1"],
                       capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode == 2
    assert "not supported" in r.stderr and "--gpus 1" in r.stderr
    assert r.stdout.strip() == ""


@pytest.mark.gpu
def test_json_line_contract():
    print("bench.py --steps 3 --warmup 1 --rows q8+:4096 --probe-gib 0.5 --no-extra", flush=True)
    r = subprocess.run([sys.executable, "-u", str(BENCH), "--steps", "3", "--warmup", "1",
                        "--rows", "q8+:4096", "--probe-gib", "0.5", "--no-extra"],
                       capture_output=True, text=True, timeout=240, cwd=ROOT)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [x for x in r.stdout.splitlines() if x.strip()]
    assert len(lines) == 1, r.stdout[-2000:]
    j = json.loads(lines[0])
    for k in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
              "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline", "checked"):
        assert k in j, k
    assert j["n_gpus"] == 1 and j["steps"] == 3 and j["warmup"] == 1
    assert j["unit"] == "tok/s" and j["higher_is_better"] is True and j["data"] == "synthetic"
    assert j["vs_baseline"] is None and j["checked"] is True
    assert "workload" in j["config"] and "model" not in j["config"]
    assert abs(j["value"] - 1000.0 / j["ms_per_step"]) <= 1e-6 * j["value"]
    rf = j["roofline"]
    for k in ("bound", "achieved", "peak", "unit", "frac", "traffic"):
        assert k in rf, k
    assert rf["bound"] == "hbm" and rf["unit"] == "GB/s" and rf["peak"] == 8000.0
    assert abs(rf["frac"] - rf["achieved"] / rf["peak"]) < 1e-9
    assert abs(rf["achieved"] - rf["algorithmic_bytes_per_launch"] / (j["ms_per_step"] * 1e6)) < 1e-6 * rf["achieved"]
    cb = j["cpu_baseline"]
    for k in ("value", "unit", "cores", "kind", "sample"):
        assert k in cb, k
    assert cb["kind"] == "port" and cb["cores"] == 1 and cb["value"] > 0
    assert j["launch_floor_us"] > 0 and j["probed_ceiling_gbps"] > 0
    assert j["device"]
    for r in j["configs"]:
        assert r["sized_ceiling_us"] > 0 and r["sized_ceiling_gbps"] > 0
        assert abs(r["mbu_sized"] - r["gbps"] / r["sized_ceiling_gbps"]) < 1e-9
