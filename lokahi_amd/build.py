"""Build libstrata_hip.so (HIP, gfx950) in-tree.

Compiles every ``csrc/*.hip`` / ``csrc/*.cpp`` with ``hipcc`` for gfx950 and
links them into ``lokahi_amd/_lib/libstrata_hip.so``.  Runs on a machine
without a GPU (hipcc cross-compiles).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT_DIR = PKG / "_lib"
LIB = OUT_DIR / "libstrata_hip.so"
PROBE_SRC = PKG / "probe" / "strata_hip_probe.cpp"
PROBE = OUT_DIR / "strata-hip-probe"  # native evidence-lane executable
INCLUDE = PKG.parent / "include"

ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.environ.get("HIPCC", f"{ROCM}/bin/hipcc")
ARCH = "gfx950"
COMMON = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed-FP32 VALU forms are disabled for all device code of this library
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # the leading kernel arguments (up to 16 dwords of pointers and scalars)
    # arrive in SGPRs with the dispatch instead of by a load at wave start
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wno-unused-result", f"-I{INCLUDE}",
]


# Per-file flags.  The prefill GEMM keeps its staging arrays in registers:
# LLVM would otherwise move them to LDS (promote-alloca), which turns every
# prefetch into a load-then-wait.
FILE_FLAGS = {
    "q4_gemm_mfma.hip": ["-mllvm", "-disable-promote-alloca-to-lds"],
}


def sources():
    return sorted(list(CSRC.glob("*.hip")) + list(CSRC.glob("*.cpp")))


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    if src.suffix == ".cpp":
        cmd[1:1] = ["-x", "hip"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{r.stderr}")


def build(verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    build_dir = OUT_DIR / "obj"
    build_dir.mkdir(exist_ok=True)
    srcs = sources()
    objs = [build_dir / (s.stem + ".o") for s in srcs]
    jobs = min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(jobs) as ex:
        futs = [ex.submit(_compile, s, o) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs),
           f"-Wl,-rpath,{ROCM}/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    tmp = PROBE.with_suffix(".tmp")
    cmd = [HIPCC, *COMMON, "-x", "hip", str(PROBE_SRC), "-o", str(tmp), f"-L{OUT_DIR}",
           "-lstrata_hip", "-Wl,-rpath,$ORIGIN"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"probe build failed:\n{r.stderr}")
    os.replace(tmp, PROBE)
    if verbose:
        print(f"built {LIB} and {PROBE.name}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
