"""The library's host code under AddressSanitizer (CPU, no GPU needed).

Every csrc/*.hip file is compiled with the host pass instrumented (device code unchanged), the
objects linked into a throw-away libnkv_amd.so in a temporary directory, and a child Python
process with the sanitizer runtime preloaded drives every host-side path that runs without a
device: the argument checks of tests/test_abi.py (each entry point rejects its bad arguments
with the expected code and message), the workspace-size functions, version and error text.
Any out-of-bounds access, use after free or double free in that host code ends the child
with the sanitizer's report, and the test fails with it.
"""
import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys
import tempfile

import pytest

from conftest import ROOT

CSRC = os.path.join(ROOT, "nanokv-llm_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"


def _asan_runtime():
    hits = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    return hits[-1] if hits else None


CHILD = r"""
import ctypes, sys, types
sys.path.insert(0, {root!r})
sys.path.insert(0, {tests!r})
sys.modules["torch"] = types.ModuleType("torch")  # the signature table only, no runtime
import importlib.util
spec = importlib.util.spec_from_file_location("nkv_lib_table", {libpy!r})
L = importlib.util.module_from_spec(spec)
spec.loader.exec_module(L)
lib = ctypes.CDLL({so!r})
for name, (res, args) in L.SIGNATURES.items():
    fn = getattr(lib, name)
    fn.restype, fn.argtypes = res, args
import test_abi
n = 0
for (name, args), code, msg in test_abi.CASES:
    rc = getattr(lib, name)(*args)
    err = lib.nkv_last_error()
    assert rc == code, (name, rc, err)
    assert msg in err, (name, err)
    n += 1
for D in (64, 128, 256):
    for bs, hq, width in ((64, 32, 32), (1, 16, 2), (500, 64, 64)):
        assert lib.nkv_paged_decode_workspace_bytes(bs, hq, D, width, 256) > 0
assert lib.nkv_paged_decode_workspace_bytes(4, 32, 96, 8, 256) == 0
assert lib.nkv_compress_select_workspace_bytes(20, 32, 8, 4, 256) > 0
assert lib.nkv_snapkv_workspace_bytes(3, 32, 8, 1024, 5) > 0
assert lib.nkv_version().startswith(b"nkv-amd")
assert "libclang_rt.asan" in open("/proc/self/maps").read()  # the runtime is live
print("host checks under the sanitizer:", n, "cases", flush=True)
"""


@pytest.mark.skipif(not os.path.exists(HIPCC) or _asan_runtime() is None,
                    reason="hipcc or the clang sanitizer runtime is not installed")
def test_host_code_under_address_sanitizer():
    sys.path.insert(0, os.path.join(ROOT, "nanokv-llm_amd"))
    import build as b  # the library's own compile flags
    out = tempfile.mkdtemp(prefix="nkv_asan_")
    try:
        host_asan = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]

        def compile_one(src):
            obj = os.path.join(out, os.path.basename(src) + ".o")
            r = subprocess.run([HIPCC, *b.HIP_FLAGS, *host_asan, "-c", src, "-o", obj],
                               capture_output=True, text=True)
            assert r.returncode == 0, r.stderr[-2000:]
            return obj

        srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
        with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
            objs = list(ex.map(compile_one, srcs))
        so = os.path.join(out, "libnkv_amd.so")
        r = subprocess.run([HIPCC, "-shared", "-fPIC", f"--offload-arch={b.ARCH}",
                            "-Xarch_host", "-fsanitize=address", "-shared-libasan", *objs,
                            "-o", so], capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-2000:]
        # the host code is instrumented: it calls the sanitizer's access checks
        syms = subprocess.run(["nm", "-D", so], capture_output=True, text=True).stdout
        assert "__asan_report_load" in syms or "__asan_loadN" in syms
        env = dict(os.environ)
        env["LD_PRELOAD"] = _asan_runtime()
        env["ASAN_OPTIONS"] = "detect_leaks=0:alloc_dealloc_mismatch=0:abort_on_error=0"
        code = CHILD.format(root=ROOT, tests=os.path.join(ROOT, "tests"), so=so,
                            libpy=os.path.join(ROOT, "nanokv-llm_amd", "_lib.py"))
        r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True,
                           env=env, timeout=300)
        assert r.returncode == 0, (r.stdout[-2000:], r.stderr[-4000:])
        assert "host checks under the sanitizer" in r.stdout
    finally:
        shutil.rmtree(out, ignore_errors=True)
