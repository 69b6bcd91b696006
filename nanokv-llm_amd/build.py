"""Build libnkv_amd.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``_build/`` (in
parallel) and linked into ``libnkv_amd.so`` next to this file, which the
ctypes loader in ``_lib.py`` opens. Runs on a machine without a GPU: hipcc
cross-compiles for gfx950. ``debug=True`` builds the same sources with
NKV_DEBUG into ``libnkv_amd_debug.so`` (objects in ``_build_debug/``): its
kernels also record the inputs they skip or clamp, read back with
nkv_debug_flags.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_NAME = "libnkv_amd.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
DEBUG_BUILD_DIR = os.path.join(PKG_DIR, "_build_debug")
DEBUG_LIB_PATH = os.path.join(PKG_DIR, "libnkv_amd_debug.so")
ARCH = os.environ.get("NKV_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
# -amdgpu-mfma-vgpr-form: MFMA accumulators stay in VGPRs, so the online-softmax
#   rescale of an accumulator needs no AGPR<->VGPR copies.
HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def _compile(hipcc: str, src: str, verbose: bool, debug: bool = False) -> str:
    obj = os.path.join(DEBUG_BUILD_DIR if debug else BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [hipcc, *HIP_FLAGS, *(["-DNKV_DEBUG"] if debug else []), "-c", src, "-o", obj]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass warns that it does not know the packed-fp32 feature.
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    return obj


def build_library(verbose: bool = False, jobs: int | None = None, debug: bool = False) -> str:
    """Compile all kernels and link libnkv_amd.so (libnkv_amd_debug.so with debug=True);
    returns its path."""
    hipcc = _hipcc()
    out = DEBUG_LIB_PATH if debug else LIB_PATH
    os.makedirs(DEBUG_BUILD_DIR if debug else BUILD_DIR, exist_ok=True)
    srcs = sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".hip"))
    jobs = jobs or min(len(srcs), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(hipcc, s, verbose, debug), srcs))
    tmp = out + ".tmp"
    cmd = [hipcc, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv, debug="--debug" in sys.argv))
