"""The C-ABI library loads and exports every function include/nkv.h declares (CPU).

No compute call is made: this container has no GPU.
"""
import ctypes
import os
import re
import subprocess

from conftest import ROOT, load_pkg

HEADER = os.path.join(ROOT, "include", "nkv.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nkv_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_path():
    names = declared_functions()
    for must in ("nkv_store_kvcache", "nkv_paged_decode", "nkv_prefill_varlen",
                 "nkv_compress_score", "nkv_compress_topk", "nkv_compress_compact",
                 "nkv_compress_finalize"):
        assert must in names


def test_library_exports_every_declared_symbol():
    load_pkg()
    from importlib import import_module
    lib_mod = import_module("nanokv-llm_amd._lib")
    lib = lib_mod.lib()
    assert os.path.exists(lib_mod.LIB_PATH)
    out = subprocess.run(["nm", "-D", "--defined-only", lib_mod.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (nkv_[a-z0-9_]+)", out))
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    # the ctypes table covers every declared function, nothing more
    assert sorted(lib_mod.SIGNATURES) == declared_functions()
    assert lib.nkv_version().startswith(b"nkv-amd")


def test_host_side_argument_checks_without_gpu():
    """Entry points reject bad arguments before touching the device."""
    from importlib import import_module
    L = import_module("nanokv-llm_amd._lib")
    lib = L.lib()
    # head_dim 64 is not supported by paged decode
    rc = lib.nkv_paged_decode_split(None, 0, None, None, None, 0, None, 1, 8, 8, 64, 256, 1, 1,
                                    1.0, None, 0, None)
    assert rc == -4 and b"head_dim" in lib.nkv_last_error()
    # top-k needs num_keep < n_cand
    rc = lib.nkv_compress_topk(None, 1, 10, 10, None, None)
    assert rc == -1 and b"num_keep" in lib.nkv_last_error()
    # zero tokens is a no-op
    assert lib.nkv_store_kvcache(None, 0, None, 0, None, None, None, 0, 8, 128, 0, None) == 0
    # workspace sizing is pure host arithmetic
    slots = (32 * 256 // 16 + 15) // 16 + 1
    assert lib.nkv_paged_decode_workspace_bytes(64, 32, 128, 32, 256) == \
        64 * 32 * slots * 130 * 4 + 64 * 32 * 4
