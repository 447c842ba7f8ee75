"""Build the gfx950 shared library lib3dmaker_amd.so in-tree with hipcc.

Every HIP/C++ source under csrc/ is compiled for gfx950 only, without FP
contraction (an FMA appears only where fmaf() is written) and with IEEE fp32
division and square root, then linked into one C-ABI shared library whose
exported symbols are declared in include/*.h.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(ROOT, "include")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "lib3dmaker_amd.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

COMMON = [
    "-O3", "-fPIC", "-std=c++17",
    f"--offload-arch={ARCH}",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA sources and results in ordinary VGPRs: no accumulation-register
    # copies between a layer's MFMAs and its epilogue
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-result", "-Wno-unused-function",
    f"-I{INCLUDE}", f"-I{CSRC}",
]


def sources():
    out = []
    for f in sorted(os.listdir(CSRC)):
        if f.endswith((".hip", ".cpp")):
            out.append(os.path.join(CSRC, f))
    return out


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON, "-c", src, "-o", obj]
    if src.endswith(".cpp"):
        cmd = [HIPCC, *COMMON, "-x", "hip", "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


PROBES_SRC = os.path.join(ROOT, "bench_probes.hip")
PROBES_LIB = os.path.join(ROOT, "bench_probes.so")


def build_probes(verbose: bool = False) -> str:
    """bench.py's device-ceiling probes, a shared library of their own (not part of the product library)."""
    tmp = PROBES_LIB + ".tmp"
    cmd = [HIPCC, *COMMON, "-shared", "-o", tmp, PROBES_SRC]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {PROBES_SRC}:\n{r.stderr}")
    os.replace(tmp, PROBES_LIB)
    if verbose:
        print(f"built {PROBES_LIB}")
    return PROBES_LIB


if __name__ == "__main__":
    build(verbose=True)
    build_probes(verbose=True)
    sys.exit(0)
