"""Builds ``libstreamindex.so`` (all HIP kernels + the C ABI) for gfx950.

The library is compiled in-tree with ``hipcc`` directly: one object per
``csrc/*.hip`` source (in parallel), then one shared-library link.  The result
lands at ``streamindex_amd/lib/libstreamindex.so`` so it travels with the
source tree to the GPU host.
"""

from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
OUT_DIR = os.path.join(PKG_DIR, "lib")
OBJ_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libstreamindex.so"
LIB_PATH = os.path.join(OUT_DIR, LIB_NAME)

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", shutil.which("hipcc") or "/opt/rocm/bin/hipcc")

# -packed-fp32-ops: keep every fp32 op scalar (no v_pk_{add,mul,fma}_f32).
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-pass-failed",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-I", CSRC,
    "-I", os.path.join(os.path.dirname(PKG_DIR), "include"),
]


# Per-source extra flags.  The sparse-attention kernel keeps its MFMA
# accumulators in VGPRs (not AGPRs): its rare online-softmax rescale multiplies
# them with VALU, and AGPR-resident accumulators made the compiler copy all of
# them into VGPRs on every loop iteration.
# The indexer units likewise: the four-M-block top-k kernel keeps its Q
# fragments in AGPRs (MFMA A-operands only) and its accumulators in VGPRs,
# where the fp32 epilogue reads them.
EXTRA_FLAGS = {
    "sparse_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    **{f"indexer_inst_{u}.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]
       for u in ("d32", "d32_wide", "d64", "d64_wide", "d128", "d128_wide", "d256",
                 "split_d32", "split_d64", "split_d128", "split_d256")},
}


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, *EXTRA_FLAGS.get(os.path.basename(src), []), "-c", src, "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}")
    return obj


def build(verbose: bool = True, jobs: int = 8) -> str:
    """Compiles every HIP source and links the shared library; returns its path."""
    os.makedirs(OUT_DIR, exist_ok=True)
    os.makedirs(OBJ_DIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    if verbose:
        print(f"[streamindex build] compiling {len(srcs)} sources for {ARCH}", flush=True)
    with cf.ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs)))) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB_PATH + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined", "-o", tmp, *objs]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[streamindex build] wrote {LIB_PATH}", flush=True)
    return LIB_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
