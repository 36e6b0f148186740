"""Build recipe for libdsa_hip.so (the gfx950 HIP kernels behind include/dsa_hip.h).

Every ``csrc/*.hip`` file is compiled with hipcc for ``--offload-arch=gfx950``
into an object under ``cppmega_amd/_build/`` and linked into
``cppmega_amd/_lib/libdsa_hip.so``.  hipcc cross-compiles without a GPU, so
this runs on any host with ROCm.  Usage: ``python -m cppmega_amd.build_lib``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_DIR = os.path.join(PKG_DIR, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libdsa_hip.so")
INCLUDE_DIR = os.path.join(os.path.dirname(PKG_DIR), "include")

ARCH = "gfx950"
# Packed fp32 VALU ops are disabled for every HIP translation unit.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]


# Per-file additions.  The indexer's epilogue is one max + one fma per score
# element, and the forward's online softmax takes a row max over every score;
# with IEEE mode off and NaN inputs declared undefined, fmaxf is a single
# v_max_f32 / v_max3_f32 instead of canonicalising each operand first (a NaN
# score still reaches the output through its exp2 term).
#
# The SparseMLA kernels keep loop-carried MFMA accumulators (O, dQ) that the
# online softmax also touches with VALU ops; LLVM's default AGPR form for MFMA
# results then copies them between AGPRs and VGPRs on every block.  The VGPR
# form keeps them in VGPRs (gfx950 MFMAs read and write either file).
_MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]
FILE_FLAGS = {
    "indexer_score.hip": ["-fno-honor-nans", "-mno-amdgpu-ieee"],
    "sparse_mla_fwd.hip": _MFMA_VGPR + ["-fno-honor-nans", "-mno-amdgpu-ieee"],
    "sparse_mla_bwd.hip": _MFMA_VGPR,
    "sparse_mla_wide.hip": _MFMA_VGPR,
    "indexer_kl_loss.hip": _MFMA_VGPR,
    "indexer_bwd.hip": _MFMA_VGPR,
}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))


def deps():
    """Every file the library is built from: the .hip sources, the kernel headers
    they include (csrc/*.hpp) and the C-ABI header (include/*.h)."""
    hdrs = [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hpp")]
    hdrs += [os.path.join(INCLUDE_DIR, f) for f in os.listdir(INCLUDE_DIR) if f.endswith(".h")]
    return sorted(sources() + hdrs)


def _compile(src: str, verbose: bool) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), f"-I{INCLUDE_DIR}", "-c", src, "-o",
           obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {os.path.basename(src)}:\n{res.stderr[-6000:]}")
    return obj


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile all kernels and link libdsa_hip.so; returns the library path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    os.makedirs(LIB_DIR, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-6000:]}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
