"""Builds libzeno.so (host engine + gfx950 HIP kernels + C ABI) and the CPU oracle.

Invoked by ``__graft_entry__.build()`` and usable directly: ``python -m zeno_amd.build``.
Every call recompiles. Objects go to ``zeno_amd/_build/``; the library lands in
``zeno_amd/libzeno.so`` and the oracle in ``oracle/libzeno_oracle.so``.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libzeno.so"
ORACLE_DIR = ROOT / "oracle"
ORACLE_LIB = ORACLE_DIR / "libzeno_oracle.so"

ARCH = os.environ.get("ZENO_AMD_ARCH", "gfx950")

# fp32 must round exactly as written: no FMA contraction, IEEE division and sqrt, no packed
# fp32 instructions.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt", "-fno-fast-math",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-result",
]
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-Wextra"]
ORACLE_FLAGS = ["-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math", "-fopenmp", "-Wall"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libzeno)")


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return res.stderr


RESOURCES = BUILD / "step_resources.txt"


def step_occupancy(remarks: str) -> dict[str, int]:
    """Waves per SIMD of each step-kernel variant, from the compiler's kernel-resource-usage
    remarks, keyed "EPW,PL,HASH" (and "EPW,PL,HASH,grouped" for the instances whose narrow
    phase visits the slots grouped by geom-type pair, "EPW,PL,HASH,split" for the instances
    with two waves per environment group). The one-environment-per-wave shapes (EPW 1) rely on
    two resident waves per SIMD to hide memory latency; a change that pushes one of them past
    256 registers can halve its throughput (the rigid pile's placement-1 kernel: 2.7x). The
    split instances need two per SIMD to hold a group's two waves on one SIMD."""
    occ, name = {}, None
    for line in remarks.splitlines():
        m = re.search(r"Function Name: \S*step_kernelILi(\d+)ELi(\d+)ELb(\d)E(?:Lb(\d)E)?(?:Lb(\d)E)?", line)
        if m:
            name = ",".join(m.groups()[:3]) + (",grouped" if m.group(4) == "1" else "") + (",split" if m.group(5) == "1" else "")
            continue
        m = re.search(r"Occupancy \[waves/SIMD\]: (\d+)", line)
        if m and name:
            occ[name] = int(m.group(1))
            name = None
    return occ


def build_oracle() -> Path:
    """Compiles the CPU oracle (test infrastructure, never linked into libzeno)."""
    cc = shutil.which("gcc") or "cc"
    tmp = ORACLE_LIB.with_suffix(".so.tmp")
    _run([cc, *ORACLE_FLAGS, str(ORACLE_DIR / "zeno_oracle.c"), "-o", str(tmp), "-lm"])
    os.replace(tmp, ORACLE_LIB)
    return ORACLE_LIB


def build_library() -> Path:
    hipcc = _hipcc()
    cxx = shutil.which("g++") or "c++"
    BUILD.mkdir(exist_ok=True)
    jobs = []
    for src in ("mjcf.cpp", "model.cpp"):
        obj = BUILD / (src + ".o")
        jobs.append([cxx, *CXX_FLAGS, "-c", str(CSRC / src), "-o", str(obj)])
    for src in ("step.hip", "world.hip", "capi.hip", "collide.hip"):
        obj = BUILD / (src + ".o")
        extra = ["-Rpass-analysis=kernel-resource-usage"] if src == "step.hip" else []
        jobs.append([hipcc, *HIP_FLAGS, *extra, "-c", str(CSRC / src), "-o", str(obj)])
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 4)) as ex:
        outs = list(ex.map(_run, jobs))
    remarks = outs[2]
    RESOURCES.write_text(remarks)
    occ = step_occupancy(remarks)
    print("step_kernel waves per SIMD (EPW,PL,HASH): " + " ".join(f"{k}={v}" for k, v in sorted(occ.items())),
          file=sys.stderr)
    objs = [str(BUILD / (s + ".o")) for s in ("mjcf.cpp", "model.cpp", "step.hip", "world.hip", "capi.hip", "collide.hip")]
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_all() -> None:
    build_library()
    build_oracle()


if __name__ == "__main__":
    build_all()
    print(f"built {LIB} and {ORACLE_LIB}", file=sys.stderr)
