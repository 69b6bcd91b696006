"""Compression scoring policy with the reference's plug-in signature.

``SnapKV(Q, K, V, num_keep, window)`` follows
nanokvllm/layers/CompressMethod.py:4-57: Q [m, Hq, window, D], K/V
[m, Hk, L, D] -> LongTensor [m, 1 + num_keep + window] =
[0, ascending top-num_keep of the key importance, L-window .. L-1], or False
when the window is too short. The importance of a key sums, over the query
window and the query heads, the softmax of the window queries' scores over
keys 0 .. L-window-1 (key 0 masked). Runs on libnkv_amd.so
(nkv_snapkv_select, or nkv_snapkv_select_f16 for fp16 Q/K: MFMA scores,
softmax, head and window sums and the top-k; window 1 with L <= 1024,
L % 64 == 0 in one fused launch, any other L through 256-key score chunks
with the last one masked). At most 4096 candidates (L - window). Scores are
fp32 (the reference computes them in the input dtype) and ties at the
selection threshold go to the lower index.
"""
from __future__ import annotations

import torch

from .. import _lib
from .compress_utils import AGG_MODES


def SnapKV(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor | None = None, num_keep: int = 220,
           window: int = 5, agg: str = "all", return_importance: bool = False):
    """Kept positions per sequence (per (sequence, KV head) with agg="group":
    [m, Hk, 1 + num_keep + window]). With return_importance the fp32 importance
    [m, n_sets, L - window] the selection was made from is returned as well."""
    m, Hk, L, D = K.shape
    Hq = Q.size(1)
    if L - window <= 0 or L <= num_keep + window:
        return False
    assert Hq % Hk == 0, f"GQA requires Hq % Hk == 0, but got Hq={Hq}, Hk={Hk}"
    _lib.require_device(K.device, Q=Q, V=V)
    f16 = _lib.is_f16(K, "SnapKV: K")
    _lib.need(K.is_contiguous() and Q.dtype == K.dtype,
              "SnapKV: Q and K must share one dtype (bf16 or fp16), K contiguous")
    _lib.need(L - window <= 4096, "SnapKV: at most 4096 candidates (L - window)")
    _lib.need(Q.shape == (m, Hq, window, D) and Q.is_contiguous(),
              f"SnapKV: Q must be contiguous [{m}, {Hq}, {window}, {D}]")
    n_sets = 1 if agg == "all" else Hk
    n_cand = L - window
    lib = _lib.lib()
    importance = torch.empty(m, n_sets, n_cand, dtype=torch.float32, device=K.device)
    keep = torch.empty(m, n_sets, num_keep + 1 + window, dtype=torch.int32, device=K.device)
    ws_bytes = lib.nkv_snapkv_workspace_bytes(m, Hq, Hk, L, window)
    workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=K.device)
    fn = lib.nkv_snapkv_select_f16 if f16 else lib.nkv_snapkv_select
    rc = fn(Q.data_ptr(), K.data_ptr(), m, Hq, Hk, D, L, window, D ** -0.5,
                               AGG_MODES[agg], num_keep, importance.data_ptr(), keep.data_ptr(),
                               workspace.data_ptr(), workspace.numel(), _lib.stream_of(K))
    _lib.check(rc, "SnapKV select")
    out = keep.to(torch.int64)
    out = out.view(m, num_keep + 1 + window) if n_sets == 1 else out
    return (out, importance) if return_importance else out
