"""Build the mpq_amd HIP library (``mpq_amd/libmpq_amd.so``) for gfx950.

Sources are compiled in-tree with hipcc, one object per translation unit, then
linked into one shared library exporting the C-ABI declared in
``include/mpq_amd.h``.  Flags:

* ``--offload-arch=gfx950`` only (no other targets, no CUDA paths);
* ``-ffp-contract=off`` so results follow the written operation order (the
  E8P12 search is bit-exact against the oracle; fmaf() is used where a fused
  multiply-add is intended);
* ``-Xclang -target-feature -Xclang -packed-fp32-ops``: no packed-FP32 VALU
  instructions are generated.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
INCLUDE = os.path.join(os.path.dirname(HERE), "include")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libmpq_amd.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)


HIP_SOURCES = [
    "e8p12_map.hip",
    "e8p12_posterior.hip",
    "gemm.hip",
    "gemm_f64.hip",
    "elementwise.hip",
    "uniform_vamp.hip",
    "e8p12_vamp.hip",
    "cd_uniform.hip",
    "e8p12_cd.hip",
    "block_cd.hip",
    "gptq_pack.hip",
    "hessian.hip",
    "awq.hip",
    "eigh.hip",
    "eigh_band.hip",
    "wy_x6.hip",
    "stedc.hip",
]
CXX_SOURCES = [
    "errors.cpp",
    "resources.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON_FLAGS = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-function",
]
# Per-file device flags.  e8p12_cd.hip: the argmin kernel seeds its MFMA accumulators from LDS and
# reads every result with VALU min operations, so accumulators in ordinary VGPRs save 32
# accumulator-register copies per 32-codeword tile; without NaN semantics the min tree needs no
# canonicalising v_max per value (the file tests finiteness on the bits where it must).
FILE_FLAGS = {
    "e8p12_cd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1", "-fno-honor-nans"],
}

HIP_FLAGS = [
    "--offload-arch=gfx950",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
]


def _run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = proc.stdout
    # hipcc's host pass does not know the packed-fp32 target feature; that warning is noise.
    lines = [ln for ln in out.splitlines() if "packed-fp32-ops" not in ln and ln.strip()]
    if proc.returncode != 0:
        raise RuntimeError("build step failed:\n  " + " ".join(cmd) + "\n" + "\n".join(lines))
    return "\n".join(lines)


def generate_sources() -> None:
    subprocess.run([sys.executable, os.path.join(CSRC, "gen_e8p12_search.py")], check=True)
    subprocess.run([sys.executable, os.path.join(CSRC, "gen_e8p12_posterior.py")], check=True)


def build(verbose: bool = False, jobs: int = 8) -> str:
    """Compile every source and link ``libmpq_amd.so``; returns the library path."""
    generate_sources()
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = []
    cmds = []
    for src in HIP_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([HIPCC, *COMMON_FLAGS, *HIP_FLAGS, *FILE_FLAGS.get(src, []), "-I", CSRC, "-I", INCLUDE, "-c",
                     os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    for src in CXX_SOURCES:
        obj = os.path.join(BUILD_DIR, src + ".o")
        cmds.append([HIPCC, *COMMON_FLAGS, "-I", CSRC, "-I", INCLUDE, "-c", os.path.join(CSRC, src), "-o", obj])
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=max(1, int(jobs))) as pool:
        for out in pool.map(_run, cmds):
            if verbose and out:
                print(out)
    tmp = LIB_PATH + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    shutil.move(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
