"""Run a test body in a child process against a comparison build of the library.

The product package always loads its own ``libvoltattn_hip.so``; a comparison
build (``voltattn_amd/build.py`` VARIANTS, e.g. the vector-ALU grouped form)
is exercised by copying the package's Python files next to the variant library
in a temporary directory and importing that copy in a fresh interpreter.

`python3 tests/variant_pkg.py stage NAME DEST` writes a self-contained copy
(package + variant library, bench.py, the oracle binding and the numerics
helper) to DEST, so a profiler can run DEST/bench.py directly against the
comparison build."""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def variant_library(name: str) -> Path:
    return ROOT / "build" / "variants" / f"libvoltattn_hip_{name}.so"


def run_child(name: str, script: Path, timeout: int = 240) -> subprocess.CompletedProcess:
    """Run `script --child` with the package copy that loads variant `name`
    first on sys.path (the repo root second, for oracle/ and tests/)."""
    lib = variant_library(name)
    if not lib.exists():
        raise FileNotFoundError(f"{lib} is not built; run `python voltattn_amd/build.py`")
    tmp = Path(tempfile.mkdtemp(prefix=f"va_{name}_"))
    try:
        pkg = tmp / "voltattn_amd"
        pkg.mkdir()
        for p in (ROOT / "voltattn_amd").glob("*.py"):
            shutil.copy(p, pkg / p.name)
        shutil.copy(lib, pkg / "libvoltattn_hip.so")
        env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(tmp), str(ROOT)]))
        env.pop("VOLTATTN_HIP_RUNTIME", None)      # the child uses no torch
        return subprocess.run([sys.executable, "-u", str(script), "--child"], cwd=ROOT, env=env,
                              capture_output=True, text=True, timeout=timeout)
    finally:
        shutil.rmtree(tmp, ignore_errors=True)


def stage(name: str, dest: Path) -> Path:
    """Copy the package (loading variant `name`), bench.py and what bench.py
    imports (oracle/, tests/numerics.py) into `dest`; returns dest/bench.py."""
    lib = variant_library(name)
    if not lib.exists():
        raise FileNotFoundError(f"{lib} is not built; run `python voltattn_amd/build.py`")
    dest = Path(dest)
    if dest.exists():
        shutil.rmtree(dest)
    for sub, files in (("voltattn_amd", sorted((ROOT / "voltattn_amd").glob("*.py"))),
                       ("oracle", [ROOT / "oracle" / f for f in ("__init__.py", "batch.py", "liboracle.so")]),
                       ("tests", [ROOT / "tests" / f for f in ("__init__.py", "numerics.py")])):
        (dest / sub).mkdir(parents=True)
        for f in files:
            shutil.copy(f, dest / sub / f.name)
    shutil.copy(lib, dest / "voltattn_amd" / "libvoltattn_hip.so")
    shutil.copy(ROOT / "bench.py", dest / "bench.py")
    return dest / "bench.py"


if __name__ == "__main__":
    if len(sys.argv) != 4 or sys.argv[1] != "stage":
        sys.exit("usage: python3 tests/variant_pkg.py stage NAME DEST")
    print(stage(sys.argv[2], Path(sys.argv[3])))
