"""Build liblogan_hip.so (gfx950) in-tree with hipcc.

Every .hip source under logan_amd/csrc is compiled to an object in parallel,
then linked into logan_amd/liblogan_hip.so. Run as a script or call build().
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "liblogan_hip.so"
INCLUDE = PKG.parent / "include"

ARCH = "gfx950"
# Packed-FP32 VALU ops stay disabled (the compiler would otherwise form
# v_pk_fma_f32 and friends from scalar float code).
HIPFLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build logan-hip)")


def _compile(src: Path, obj_dir: Path = OBJ, defines: tuple = ()) -> Path:
    out = obj_dir / (src.stem + ".o")
    cmd = [hipcc(), *HIPFLAGS, *(f"-D{d}" for d in defines), "-I", str(INCLUDE), "-c", str(src),
           "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")
    return out


# The stage-timeline variant of the library (moe_fused.hip built with
# LOGAN_HIP_TIMELINE; see logan_amd/timeline.py). Never loaded unless named.
TIMELINE_OBJ = PKG / "_build_tl"
TIMELINE_LIB = PKG / "liblogan_hip_timeline.so"


def build(verbose: bool = False, timeline: bool = False) -> Path:
    obj_dir, lib, defines = (TIMELINE_OBJ, TIMELINE_LIB, ("LOGAN_HIP_TIMELINE",)) if timeline \
        else (OBJ, LIB, ())
    obj_dir.mkdir(exist_ok=True)
    srcs = sorted(CSRC.glob("*.hip"))
    if not srcs:
        raise RuntimeError("no HIP sources found")
    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        objs = list(ex.map(lambda src: _compile(src, obj_dir, defines), srcs))
    tmp = lib.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, lib)
    if verbose:
        print(f"built {lib}")
    return lib


if __name__ == "__main__":
    build(verbose=True, timeline="--timeline" in sys.argv[1:])
    sys.exit(0)
