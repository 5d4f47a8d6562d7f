"""CPU: the fused merge's ticket-slot binding (voltattn_amd/csrc/va_slots.hpp).

Calls on one stream run one after another and may share a ticket slot; calls
on different streams (or a captured graph and anything else) must not. The
binding logic is plain C++, so tests/cpp/test_slots.cpp drives it directly:
one slot per eager stream, one per (stream, capture sequence), distinct
slots across streams and captures, per-device tables, -1 (two-pass form) once
a device's 16 slots are bound and none can be taken over, distinct slots under
concurrent first calls from 16 threads; a take-over only of an idle eager
owner with no call between acquire() and done(), never of a capture's slot;
call counters that outlive bindings; and, under concurrent take-overs by 8
threads sharing 2 slots, never two calls holding one slot."""
import subprocess
import tempfile
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent


def test_slot_binding():
    with tempfile.TemporaryDirectory() as d:
        exe = Path(d) / "test_slots"
        subprocess.run(["g++", "-O1", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-pthread",
                        "-I", str(ROOT / "voltattn_amd" / "csrc"), str(ROOT / "tests" / "cpp" / "test_slots.cpp"),
                        "-o", str(exe)], check=True)
        r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0, r.stderr
        assert "slots: ok" in r.stdout
