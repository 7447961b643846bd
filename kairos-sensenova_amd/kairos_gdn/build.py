"""Build libkairos_gdn.so (the HIP kernels + C ABI) for gfx950 with hipcc.

Each csrc/*.hip translation unit is compiled in parallel and linked into
kairos_gdn/libkairos_gdn.so next to this file.  Works without a GPU (hipcc
cross-compiles).  Usage: ``python kairos-sensenova_amd/kairos_gdn/build.py``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
SRC_DIR = os.path.join(os.path.dirname(PKG_DIR), "csrc")
INCLUDE_DIR = os.path.join(os.path.dirname(os.path.dirname(PKG_DIR)), "include")
BUILD_DIR = os.path.join(os.path.dirname(PKG_DIR), "_build")
LIB_NAME = "libkairos_gdn.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
# gfx950 only: the kernels use its OCP fp8 decode, 16-bit transposed LDS reads and 160 KB of LDS
# per CU (gdn_common.hpp also refuses device code for any other target).
ARCH = "gfx950"
if os.environ.get("KAIROS_GDN_ARCH", ARCH) != ARCH:
    raise RuntimeError(f"KAIROS_GDN_ARCH={os.environ['KAIROS_GDN_ARCH']}: libkairos_gdn is built for gfx950 only")

# -packed-fp32-ops: keep the compiler from forming packed fp32 VALU ops (the
# host pass warns that it does not know the feature; that is harmless).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-file flags.  MFMA accumulators in VGPRs: the fused K = 256 kernel scales and packs its state with
# VALU every chunk (in AGPRs each of those touches costs a copy); the segment scan's kernels measured
# alike at config 2 and 0.8% faster on the streaming rollout, the backward's 0.2% faster at the layer
# shape (A/B in one GPU call).
FILE_FLAGS = {
    "gdn_wide.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gdn_seg.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "gdn_bwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(exe):
        raise RuntimeError("hipcc not found: the HIP toolchain (ROCm) is required to build libkairos_gdn.so")
    return exe


def sources():
    return sorted(os.path.join(SRC_DIR, f) for f in os.listdir(SRC_DIR) if f.endswith(".hip"))


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src)[:-4] + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *FILE_FLAGS.get(os.path.basename(src), []), "-I", INCLUDE_DIR, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every kernel source and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
