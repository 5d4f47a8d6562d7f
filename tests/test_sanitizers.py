"""CPU: the host code under AddressSanitizer + UndefinedBehaviorSanitizer.

* The C ABI unit's host code (va_runtime.hip: validation, size rules, slot
  binding, error paths) from the comparison build
  build/variants/libvoltattn_hip_hostsan.so (hipcc, each -fsanitize= given to
  the host compilation only), driven by the CPU suite's ABI and torch-op tests
  in a child process with clang's ASan runtime preloaded.
* The oracle (oracle/oracle.cpp), rebuilt here with g++ -fsanitize=address,
  undefined, driven by its own CPU tests (draws, fp16, quantizer, reference,
  the reference's logged selftest fingerprints, planted mistakes) with gcc's
  ASan runtime preloaded.
* The C++ harness (tests/cli/voltattn_cli.cpp) and the oracle built into one
  sanitized executable, running its host-only selftest (--selftest-host: every
  case's inputs, quantizer, double reference and split-merge algebra).
* The ticket-slot table (tests/cpp/test_slots.cpp) under ASan+UBSan and under
  ThreadSanitizer (its concurrent first-call case).
Any sanitizer report fails the run (-fno-sanitize-recover, ASan aborts)."""
import os
import shutil
import subprocess
import sys
import tempfile
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SAN = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g", "-O1"]
ENV_ASAN = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def _gcc_rt(name: str) -> str:
    return subprocess.run(["g++", f"-print-file-name={name}"], capture_output=True, text=True, check=True).stdout.strip()


def _clang_asan_rt() -> Path:
    hits = sorted(Path("/opt/rocm/llvm/lib/clang").glob("*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not hits:
        pytest.skip("clang's ASan runtime is not installed")
    return hits[-1]


def _run(cmd, env=None, timeout=600, cwd=None):
    e = dict(os.environ)
    e.pop("VOLTATTN_HIP_RUNTIME", None)
    e.update(env or {})
    r = subprocess.run(cmd, capture_output=True, text=True, env=e, timeout=timeout, cwd=cwd)
    assert r.returncode == 0, f"{cmd}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
    return r


def _pytest_child(pkg_dir: Path, module: str, tests, preload: str) -> str:
    """Run pytest on `tests` in a child whose `module` is the copy in pkg_dir."""
    code = (f"import sys; import {module} as m; assert str(m.LIB_PATH).startswith({str(pkg_dir)!r}), m.LIB_PATH; "
            f"import pytest; sys.exit(pytest.main(['-q', '-p', 'no:cacheprovider', '--import-mode=append', "
            f"'-m', 'not gpu', *{[str(t) for t in tests]!r}]))")
    env = dict(ENV_ASAN, LD_PRELOAD=preload, PYTHONPATH=os.pathsep.join([str(pkg_dir), str(ROOT)]))
    return _run([sys.executable, "-c", code], env=env, cwd=pkg_dir).stdout     # cwd: the copy wins


def test_c_abi_host_code_under_asan_ubsan():
    lib = ROOT / "build" / "variants" / "libvoltattn_hip_hostsan.so"
    if not lib.exists():
        pytest.fail(f"{lib} is not built; run `python voltattn_amd/build.py`")
    with tempfile.TemporaryDirectory() as d:
        pkg = Path(d) / "voltattn_amd"
        pkg.mkdir()
        for p in (ROOT / "voltattn_amd").glob("*.py"):
            shutil.copy(p, pkg / p.name)
        shutil.copy(lib, pkg / "libvoltattn_hip.so")
        out = _pytest_child(Path(d), "voltattn_amd",
                            [ROOT / "tests" / f for f in ("test_abi.py", "test_abi_batch.py", "test_torch_ops.py")],
                            str(_clang_asan_rt()))
        assert " passed" in out and "failed" not in out, out[-2000:]


def test_oracle_under_asan_ubsan():
    with tempfile.TemporaryDirectory() as d:
        pkg = Path(d) / "oracle"
        pkg.mkdir()
        for p in (ROOT / "oracle").glob("*.py"):
            shutil.copy(p, pkg / p.name)
        _run(["g++", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off", "-pthread", "-Wall", "-Wextra",
              "-Werror", *SAN, str(ROOT / "oracle" / "oracle.cpp"), "-o", str(pkg / "liboracle.so")])
        tests = sorted((ROOT / "tests").glob("test_oracle_*.py")) + [ROOT / "tests" / "test_fingerprints.py",
                                                                     ROOT / "tests" / "test_negative.py"]
        out = _pytest_child(Path(d), "oracle", tests, _gcc_rt("libasan.so"))
        assert " passed" in out and "failed" not in out, out[-2000:]


def test_cli_host_selftest_under_asan_ubsan():
    lib = ROOT / "voltattn_amd" / "libvoltattn_hip.so"
    with tempfile.TemporaryDirectory() as d:
        exe = Path(d) / "voltattn_san"
        _run(["g++", "-std=c++17", "-pthread", "-Wall", "-Wextra", "-Werror", "-ffp-contract=off", *SAN,
              "-I", str(ROOT / "include"), "-I", str(ROOT / "oracle"), "-I", str(ROOT / "voltattn_amd" / "host"),
              str(ROOT / "tests" / "cli" / "voltattn_cli.cpp"), str(ROOT / "oracle" / "oracle.cpp"),
              "-o", str(exe), f"-L{lib.parent}", "-lvoltattn_hip", f"-Wl,-rpath,{lib.parent}"])
        out = _run([str(exe), "--selftest-host"], env=ENV_ASAN).stdout
        assert "host selftest: all 72 cases ok" in out, out[-2000:]


@pytest.mark.parametrize("flags", [SAN, ["-fsanitize=thread", "-g", "-O1"]], ids=["asan-ubsan", "tsan"])
def test_slot_table_under_sanitizers(flags):
    with tempfile.TemporaryDirectory() as d:
        exe = Path(d) / "test_slots"
        _run(["g++", "-std=c++17", "-pthread", "-Wall", "-Wextra", "-Werror", *flags,
              "-I", str(ROOT / "voltattn_amd" / "csrc"), str(ROOT / "tests" / "cpp" / "test_slots.cpp"),
              "-o", str(exe)])
        out = _run([str(exe)], env=dict(ENV_ASAN, TSAN_OPTIONS="halt_on_error=1")).stdout
        assert "slots: ok" in out
