"""ctypes binding of libnkv_amd.so (declared in include/nkv.h).

The library is the only compute path of this package: if it is missing the
loader raises, there is no CPU or PyTorch fallback. With NKV_DEBUG=1 in the
environment the loader opens libnkv_amd_debug.so instead (the same kernels
built with NKV_DEBUG, which also record the inputs they skip or clamp; see
debug_flags). torch is imported first
so that the HIP runtime torch ships (SONAME libamdhip64.so.7) is the one the
library binds to; the streams handed over are torch's own.
"""
from __future__ import annotations

import ctypes as C
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "libnkv_amd.so")
DEBUG_LIB_PATH = os.path.join(PKG_DIR, "libnkv_amd_debug.so")

NKV_OK = 0
NKV_AGG_ALL = 0
NKV_AGG_GROUP = 1
NKV_DECODE_NOALLOC_MAX_BYTES = 64 << 20  # include/nkv.h
NKV_DEBUG_SLOT = 1  # include/nkv.h: bits of nkv_debug_flags
NKV_DEBUG_BLOCK = 2
NKV_DEBUG_LENGTH = 4
NKV_DEBUG_POSITION = 8

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float
_sz = C.c_size_t

# name -> (restype, argtypes); mirrors include/nkv.h
SIGNATURES = {
    "nkv_last_error": (C.c_char_p, []),
    "nkv_version": (C.c_char_p, []),
    "nkv_debug_flags": (C.c_int, [_p, _i32]),
    "nkv_store_kvcache": (C.c_int, [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i32, _i32, _i64, _p]),
    "nkv_fp8_quantize": (C.c_int, [_p, _i64, _f32, _p, _p]),
    "nkv_fp8_dequantize": (C.c_int, [_p, _i64, _f32, _p, _p]),
    "nkv_store_kvcache_fp8": (C.c_int, [_p, _i64, _p, _i64, _p, _p, _p, _i64, _i32, _i32, _i64,
                                        _f32, _f32, _p]),
    "nkv_qk_norm_rope_store": (C.c_int, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _f32, _p,
                                         _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i32,
                                         _i32, _i32, _p]),
    "nkv_qk_norm_rope_store_f16": (C.c_int, [_p, _i64, _p, _i64, _p, _i64, _p, _p, _p, _f32, _p,
                                             _i64, _p, _i64, _p, _p, _p, _p, _i64, _i64, _i32,
                                             _i32, _i32, _p]),
    "nkv_paged_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "nkv_paged_decode": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32,
                                   _i32, _i64, _f32, _p, _i64, _p, _sz, _p]),
    "nkv_paged_decode_noalloc": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _p, _i32, _i32, _i32,
                                           _i32, _i32, _i32, _i64, _f32, _p, _i64, _p]),
    "nkv_paged_decode_f16": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32,
                                       _i32, _i32, _i64, _f32, _p, _i64, _p, _sz, _p]),
    "nkv_paged_decode_fp8": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32,
                                       _i32, _i32, _i64, _f32, _f32, _f32, _p, _i64, _p, _sz,
                                       _p]),
    "nkv_paged_decode_split": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32,
                                         _i32, _i32, _i64, _f32, _p, _sz, _p]),
    "nkv_paged_decode_combine": (C.c_int, [_p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _i64, _p,
                                           _sz, _p]),
    "nkv_prefill_varlen": (C.c_int, [_p, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _i32, _i64, _f32, _p, _i64, _p]),
    "nkv_prefill_varlen_f16": (C.c_int, [_p, _i64, _p, _p, _i64, _i64, _p, _p, _p, _i64, _i32,
                                         _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32, _p,
                                         _i64, _p]),
    "nkv_prefill_varlen_fp8": (C.c_int, [_p, _i64, _p, _p, _p, _p, _p, _i64, _i32, _i32, _i32,
                                         _i32, _i32, _i32, _i32, _i64, _f32, _f32, _f32, _p,
                                         _i64, _p]),
    "nkv_compress_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32]),
    "nkv_compress_score": (C.c_int, [_p, _i64, _p, _p, _i64, _i32, _p, _p, _i32, _i32, _i32, _i32,
                                     _i32, _i32, _i64, _f32, _i32, _p, _p, _sz, _p]),
    "nkv_compress_topk": (C.c_int, [_p, _i32, _i32, _i32, _p, _p]),
    "nkv_compress_select_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "nkv_compress_select": (C.c_int, [_p, _i64, _p, _p, _i64, _i32, _p, _p, _i32, _i32, _i32,
                                      _i32, _i32, _i32, _i64, _f32, _i32, _i32, _p, _p, _p, _sz,
                                      _p]),
    "nkv_compress_select_f16": (C.c_int, [_p, _i64, _p, _p, _i64, _i32, _p, _p, _i32, _i32, _i32,
                                          _i32, _i32, _i32, _i64, _f32, _i32, _i32, _p, _p, _p,
                                          _sz, _p]),
    "nkv_snapkv_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32]),
    "nkv_snapkv_select": (C.c_int, [_p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32,
                                    _p, _p, _p, _sz, _p]),
    "nkv_snapkv_select_f16": (C.c_int, [_p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _i32,
                                        _i32, _p, _p, _p, _sz, _p]),
    "nkv_compress_step": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p, _i32, _i32, _i32,
                                    _i32, _i32, _i32, _i64, _f32, _i32, _i32, _p, _p, _p, _sz,
                                    _p]),
    "nkv_compress_step_f16": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p, _i32, _i32,
                                        _i32, _i32, _i32, _i32, _i64, _f32, _i32, _i32, _p, _p,
                                        _p, _sz, _p]),
    "nkv_compress_step_fp8": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p, _i32, _i32,
                                        _i32, _i32, _i32, _i32, _i64, _f32, _f32, _i32, _i32, _p,
                                        _p, _p, _sz, _p]),
    "nkv_compress_step_finalize": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p, _i32,
                                             _i32, _i32, _i32, _i32, _i32, _i64, _f32, _i32,
                                             _i32, _p, _p, _p, _sz, _i32, _p, _p, _p]),
    "nkv_compress_step_finalize_f16": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p,
                                                 _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32,
                                                 _i32, _i32, _p, _p, _p, _sz, _i32, _p, _p, _p]),
    "nkv_compress_step_finalize_fp8": (C.c_int, [_p, _i64, _p, _p, _p, _i64, _i32, _p, _p, _p,
                                                 _i32, _i32, _i32, _i32, _i32, _i32, _i64, _f32,
                                                 _f32, _i32, _i32, _p, _p, _p, _sz, _i32, _p, _p,
                                                 _p]),
    "nkv_compress_compact": (C.c_int, [_p, _p, _p, _i64, _i32, _p, _p, _p, _i32, _p, _i32, _i32,
                                       _i32, _i32, _i32, _i32, _i64, _p]),
    "nkv_compress_finalize": (C.c_int, [_p, _i64, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _p,
                                        _p, _p]),
    "nkv_compress_schedule": (C.c_int, [_p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _p, _p, _p,
                                        _p, _p]),
    "nkv_build_step_metadata": (C.c_int, [_p, _i32, _i32, _i32, _i64, _i32, _p, _i64, _i32, _i32,
                                          _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i32, _p]),
}

_LIB = None


class NkvError(RuntimeError):
    pass


def lib_path() -> str:
    """libnkv_amd.so, or libnkv_amd_debug.so when NKV_DEBUG=1 is set."""
    return DEBUG_LIB_PATH if os.environ.get("NKV_DEBUG") == "1" else LIB_PATH


def lib() -> C.CDLL:
    """Load the library once; raise if it has not been built."""
    global _LIB
    if _LIB is None:
        path = lib_path()
        if not os.path.exists(path):
            raise NkvError(
                f"{path} is missing: build it with `python __graft_entry__.py build` "
                "(or nanokv-llm_amd/build.py); there is no fallback path")
        handle = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = handle
    return _LIB


def debug_flags(clear: bool = True) -> int:
    """NKV_DEBUG_* bits the debug library's kernels recorded on the current device since
    the last clearing call (waits for the device). Raises NkvError with the release
    library, which records nothing."""
    v = C.c_uint32(0)
    check(lib().nkv_debug_flags(C.addressof(v), 1 if clear else 0), "debug_flags")
    return v.value


def check(rc: int, what: str) -> None:
    if rc != NKV_OK:
        msg = lib().nkv_last_error().decode(errors="replace")
        raise NkvError(f"{what} failed (code {rc}): {msg}")


def require_device(device: torch.device, **tensors: torch.Tensor | None) -> None:
    """The kernels take raw device pointers: every tensor given must be a GPU tensor on
    ``device`` (None entries are skipped). Raises ValueError naming the first that is not,
    before anything reaches the library."""
    if device.type != "cuda":
        raise ValueError(f"expected GPU tensors, got a tensor on {device}")
    for name, t in tensors.items():
        if t is not None and t.device != device:
            raise ValueError(f"{name} is on {t.device}, expected {device}")


def is_f16(t: torch.Tensor, what: str) -> bool:
    """Activations (q, k, v, outputs) and 16-bit caches are bf16 or fp16, as the model's
    dtype: True for fp16 (the kernels' _f16 entry points), False for bf16; raises otherwise."""
    if t.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError(f"{what} must be bf16 or fp16, got {t.dtype}")
    return t.dtype == torch.float16


def need(cond: bool, msg: str) -> None:
    """Argument check that survives ``python -O``: raises ValueError(msg)."""
    if not cond:
        raise ValueError(msg)


def stream_of(t: torch.Tensor) -> int:
    """HIP stream handle of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
