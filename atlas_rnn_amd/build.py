"""Ahead-of-time build of libatlas_mem.so for gfx950 (hipcc, no JIT, no torch extension).

    python -m atlas_rnn_amd.build          # builds atlas_rnn_amd/libatlas_mem.so in place

The library is plain HIP C++ with an extern "C" ABI (include/atlas_mem.h); the Python package
loads it with ctypes.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
LIB_NAME = "libatlas_mem.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["abi.hip", "coef.hip", "seg_fwd.hip", "seg_bwd.hip", "scan.hip", "affine.hip", "bwd_scalar.hip", "walk_fwd.hip", "walk_bwd.hip", "tmap.hip", "step.hip", "prologue.hip", "blocks.hip", "factors.hip", "bufwalk.hip", "wgrad.hip", "gemm.hip", "chunk_bwd.hip", "chunk_coef.hip"]
ARCH = os.environ.get("ATLAS_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    # keep the compiler from forming packed fp32 ops (v_pk_{add,mul,fma}_f32)
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{os.path.join(ROOT, 'include')}",
]


# Per-source options. The ILP-first machine schedulers keep more independent LDS reads and matrix
# products in flight in two kernels bound by latency at two waves per SIMD: the reverse chunk walk
# (k_cp_bwd, iterative ILP: -1.5 to -2.4 % in same-box measurements) and the adjoint aggregates
# (k_bwd_seg_agg, max ILP: -2 to -5 %). Kernels measured slower with either keep the default (k_tmap_fwd,
# k_tmap_bwd, k_walk_full, k_walk_agg). The tensor map's kernels take the scheduler's own AMDGPU
# register-pressure trackers instead (fewer spills in k_tmap_fwd, 64 -> 48; both kernels -3 to -4 %).
SOURCE_FLAGS = {
    "chunk_bwd.hip": ["-mllvm", "-amdgpu-sched-strategy=iterative-ilp"],
    "seg_bwd.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "tmap.hip": ["-mllvm", "-amdgpu-use-amdgpu-trackers"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libatlas_mem.so)")


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 and link libatlas_mem.so. Always recompiles."""
    hipcc = _hipcc()
    obj_dir = os.path.join(PKG_DIR, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES:
        obj = os.path.join(obj_dir, src.replace(".hip", ".o"))
        objs.append(obj)
        cmds.append([hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj])
    with ThreadPoolExecutor(max_workers=min(len(cmds), max(1, (os.cpu_count() or 2) // 2))) as ex:
        list(ex.map(lambda c: _run(c, verbose), cmds))
    tmp = LIB_PATH + ".tmp"
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
