"""Build the in-tree native libraries of qw3_amd.

    libds3_hip.so  HIP kernels (gfx950) + the C-ABI host runtime (include/ds3_hip.h)
    libds3gen.so   synthetic workload generator / GGUF block quantisers (host C)

Both land in qw3_amd/lib/.  Object files go to qw3_amd/_build/.  Every call
recompiles (the driver's build check); translation units compile in parallel.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "lib"
BUILD = PKG / "_build"
ARCH = os.environ.get("DS3_HIP_ARCH", "gfx950")

HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    # packed fp32 instructions stay off ("Build")
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; drop that noise
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build step failed ({r.returncode}): {' '.join(cmd)}\n{r.stdout}\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build_gen() -> Path:
    LIB.mkdir(exist_ok=True)
    out = LIB / "libds3gen.so"
    _run(["gcc", "-O2", "-fPIC", "-shared", "-std=c11", "-Wall", "-Wextra",
          str(CSRC / "gen" / "ds3_gen.c"), "-o", str(out), "-lm", "-lpthread"])
    return out


def build_hip(jobs: int | None = None) -> Path:
    LIB.mkdir(exist_ok=True)
    BUILD.mkdir(exist_ok=True)
    srcs = [CSRC / "ds3_hip.cpp"] + sorted((CSRC / "kernels").glob("*.hip"))
    objs = [BUILD / (s.stem + ".o") for s in srcs]
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-x", "hip", "-c", str(s), "-o", str(o)])
                for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    out = LIB / "libds3_hip.so"
    tmp = LIB / "libds3_hip.so.tmp"
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, out)
    return out


def build_all() -> None:
    build_gen()
    build_hip()


if __name__ == "__main__":
    build_all()
    print("built:", *sorted(p.name for p in LIB.glob("*.so")))
