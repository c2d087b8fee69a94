"""Builds the HIP library (gfx950) in-tree, and the CPU oracle used by tests.

    python -m inferno_amd._build
"""
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "inferno_amd"
CSRC = PKG / "csrc"
LIB = PKG / "libinferno_moe.so"
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "liboracle.so"
BUILD_DIR = ROOT / "build" / "obj"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 ops stay off: hand-free code must not emit v_pk_*_f32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(map(str, cmd))}\n{r.stdout}\n{r.stderr}")
    return r


def build_hip():
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    objs = [BUILD_DIR / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        list(ex.map(lambda so: _run([HIPCC, *HIP_FLAGS, "-c", str(so[0]), "-o", str(so[1])]),
                    zip(srcs, objs)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
          "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"])
    os.replace(tmp, LIB)
    return LIB


def build_oracle():
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run(["g++", "-O3", "-std=c++17", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared",
          "-pthread", "-o", str(tmp), str(ORACLE_DIR / "oracle.cpp")])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_all():
    with cf.ThreadPoolExecutor(max_workers=2) as ex:
        a = ex.submit(build_hip)
        b = ex.submit(build_oracle)
        return a.result(), b.result()


if __name__ == "__main__":
    for p in build_all():
        print(p)
    sys.exit(0)
