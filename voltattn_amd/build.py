"""Build recipe for the in-tree native artefacts.

    python voltattn_amd/build.py            # library + oracle + CLI harness

(run as a file, not ``-m``: importing the package loads the library being built)

* ``voltattn_amd/libvoltattn_hip.so`` — the product: gfx950 HIP kernels and the
  C ABI of ``include/voltattn.h`` (hipcc, one object per ``csrc/*.hip``).
* ``build/variants/libvoltattn_hip_valu.so`` — the same library with the
  grouped-query q8/q4 kernels in their vector-ALU form (``VA_GQA_MFMA=0``):
  the comparison build ``tests/test_gpu_valu_form.py`` runs. Only
  ``va_decode_ex.hip`` differs; the other objects are the product's.
* ``build/variants/libvoltattn_hip_hostsan.so`` — the C ABI unit
  (``va_runtime.hip``) with its host code built under AddressSanitizer and
  UndefinedBehaviorSanitizer (device code unchanged), for the CPU sanitizer
  run of ``tests/test_sanitizers.py``.
* ``oracle/liboracle.so`` — the CPU checker (test infrastructure, g++).
* ``build/voltattn`` — the C++ selftest/bench/probe harness (tests/cli), linked
  against both.

Everything is compiled every time (the driver's "does it build" check); objects
go to ``build/obj`` and the shared library is replaced atomically.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "voltattn_amd"
CSRC = PKG / "csrc"
OBJ = ROOT / "build" / "obj"
LIB = PKG / "libvoltattn_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wextra",
    "-Werror",
    "-Wno-unused-command-line-argument",
    # Keep hipcc from forming packed-FP32 (v_pk_*_f32) instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in arch VGPRs (the matrix-core decode fits in 256 of
    # them); the AGPR form shuttled them through v_accvgpr moves.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # Kernel argument preload: the first 16 dwords of scalar kernel arguments
    # arrive in SGPRs with the wave (the code object keeps a prologue that
    # loads them itself where the firmware does not preload).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


# Per-unit exceptions to HIPCC_FLAGS. The read probes lose ~1.2 us per launch
# with kernel argument preload (MI355X, a 142.6 MB chunked read: 22.2 ->
# 23.4 us back to back); their arguments are few and needed late.
UNIT_DROP_FLAGS = {
    "va_probe.hip": ("-amdgpu-kernarg-preload-count=16",),
}


def unit_flags(src: Path) -> list[str]:
    drop = UNIT_DROP_FLAGS.get(Path(src).name, ())
    out: list[str] = []
    for f in HIPCC_FLAGS:
        if f in drop:
            out.pop()            # the "-mllvm" in front of it
            continue
        out.append(f)
    return out


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build voltattn_amd)")


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    res = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


VARIANTS = {
    # name: (translation unit(s) rebuilt, their defines, their extra compiler flags)
    "valu": ("va_decode_ex.hip", ("VA_GQA_MFMA=0",), ()),
    # test only: every fused merge gives up after its bounded wait (NaN output,
    # counted for va_merge_faults), so the failure path runs with kernels that
    # all exit normally
    "lost": (("va_decode.hip", "va_decode_ex.hip"), ("VA_TEST_LOSE_MERGES=1",), ()),
    # host code only: each -fsanitize= goes to the host compilation
    "hostsan": ("va_runtime.hip", (), ("-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                                       "-Xarch_host", "-fno-sanitize-recover=all", "-Xarch_host", "-fno-omit-frame-pointer",
                                       "-Xarch_host", "-g")),
}
VARIANT_LINK = {"hostsan": ("-fsanitize=address", "-fsanitize=undefined")}
VARIANT_DIR = ROOT / "build" / "variants"


def variant_path(name: str) -> Path:
    return VARIANT_DIR / f"libvoltattn_hip_{name}.so"


def _link(cc: str, objs, out: Path, flags=()) -> Path:
    out = Path(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *flags, "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, out)
    return out


def build_library(jobs: int = 8, out: Path = LIB, defines: tuple[str, ...] = (),
                  variants: tuple[str, ...] = ()) -> Path:
    """Compile csrc/*.hip and link `out`; `defines` (e.g. "VA_LOAD_AUX=2") build a
    variant of the whole library; `variants` (names in VARIANTS) also link those
    comparison libraries from the same objects plus their rebuilt unit."""
    obj_dir = OBJ if not defines else OBJ / ("v_" + "_".join(d.replace("=", "") for d in defines))
    obj_dir.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    cc = hipcc()
    dflags = [f"-D{d}" for d in defines]
    jobs_list = [(src, obj_dir / (src.stem + ".o"), dflags) for src in srcs]
    vjobs = {}
    for name in variants:
        units, vdefs, vflags = VARIANTS[name]
        units = (units,) if isinstance(units, str) else units
        vdir = obj_dir / f"variant_{name}"
        vdir.mkdir(parents=True, exist_ok=True)
        vjobs[name] = []
        for unit in units:
            vjobs[name].append(len(jobs_list))
            jobs_list.append((CSRC / unit, vdir / (Path(unit).stem + ".o"),
                              dflags + [f"-D{d}" for d in vdefs] + list(vflags)))

    def compile_one(job) -> Path:
        src, obj, fl = job
        _run([cc, *unit_flags(src), *fl, "-I", str(ROOT / "include"), "-c", str(src), "-o", str(obj)])
        return obj

    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        objs = list(ex.map(compile_one, jobs_list))
    main_objs = objs[:len(srcs)]
    _link(cc, main_objs, out)
    for name in variants:
        rebuilt = [objs[i] for i in vjobs[name]]
        stems = {o.stem for o in rebuilt}
        vobjs = [o for o in main_objs if o.stem not in stems] + rebuilt
        _link(cc, vobjs, variant_path(name), VARIANT_LINK.get(name, ()))
    return Path(out)


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "liboracle.so"


def build_cli() -> Path:
    out = ROOT / "build" / "voltattn"
    out.parent.mkdir(parents=True, exist_ok=True)
    tmp = out.with_name("voltattn.tmp")
    _run([
        "g++", "-O2", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-pthread",
        "-I", str(ROOT / "include"), "-I", str(ROOT / "oracle"), "-I", str(PKG / "host"),
        str(ROOT / "tests" / "cli" / "voltattn_cli.cpp"),
        "-o", str(tmp),
        f"-L{PKG}", "-lvoltattn_hip", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,$ORIGIN/../voltattn_amd",
        f"-L{ROOT / 'oracle'}", "-loracle", f"-Wl,-rpath,{ROOT / 'oracle'}",
        "-Wl,-rpath,$ORIGIN/../oracle",
    ])
    os.replace(tmp, out)
    return out


def build_all(jobs: int = 8) -> None:
    build_library(jobs, variants=tuple(VARIANTS))
    build_oracle()
    if (ROOT / "tests" / "cli" / "voltattn_cli.cpp").exists():
        build_cli()


if __name__ == "__main__":
    build_all(int(sys.argv[1]) if len(sys.argv) > 1 else 8)
    print(f"built {LIB}")
