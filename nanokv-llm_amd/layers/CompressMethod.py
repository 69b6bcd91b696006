"""Compression scoring policy with the reference's plug-in signature.

``SnapKV(Q, K, V, num_keep, window)`` follows
nanokvllm/layers/CompressMethod.py:4-57: Q [m, Hq, window, D], K/V
[m, Hk, L, D] -> LongTensor [m, 1 + num_keep + window] =
[0, ascending top-num_keep of the key importance, L-window .. L-1], or False
when the window is too short. Runs on libnkv_amd.so (nkv_compress_select:
MFMA scores, softmax, head sum and top-k in one launch for L <= 1024, L % 64
== 0; otherwise L % 256 == 0 is required); scores are fp32 (the reference computes them in bf16) and ties at the
selection threshold go to the lower index.
"""
from __future__ import annotations

import torch

from .. import _lib
from .compress_utils import AGG_MODES


def SnapKV(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor | None = None, num_keep: int = 220,
           window: int = 5, agg: str = "all"):
    m, Hk, L, D = K.shape
    Hq = Q.size(1)
    if L - window <= 0 or L <= num_keep + window:
        return False
    if window != 1:
        raise NotImplementedError("SnapKV on libnkv_amd supports window=1 (the periodic "
                                  "compression step's latest-token query)")
    assert Hq % Hk == 0, f"GQA requires Hq % Hk == 0, but got Hq={Hq}, Hk={Hk}"
    assert K.is_contiguous() and K.dtype == torch.bfloat16 and Q.dtype == torch.bfloat16
    assert Q.size(2) == 1 and Q.stride(1) == D and Q.stride(3) == 1
    n_sets = 1 if agg == "all" else Hk
    n_cand = L - 1
    lib = _lib.lib()
    importance = torch.empty(m, n_sets, n_cand, dtype=torch.float32, device=K.device)
    keep = torch.empty(m, n_sets, num_keep + 2, dtype=torch.int32, device=K.device)
    ws_bytes = lib.nkv_compress_select_workspace_bytes(m, Hq, Hk, 1, L)
    workspace = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=K.device)
    # contiguous K: one "block" of L tokens per (sequence, KV head)
    rc = lib.nkv_compress_select(Q.data_ptr(), Q.stride(0), K.data_ptr(), None, 0, 0, None,
                                 None, m, Hq, Hk, D, L, 1, 0, D ** -0.5, AGG_MODES[agg],
                                 num_keep, importance.data_ptr(), keep.data_ptr(),
                                 workspace.data_ptr(), workspace.numel(), _lib.stream_of(K))
    _lib.check(rc, "SnapKV select")
    out = keep.to(torch.int64)
    return out.view(m, num_keep + 2) if n_sets == 1 else out
