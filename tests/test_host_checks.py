"""Host-side argument checks of the Python wrappers (no GPU needed).

The library takes raw device pointers, so a host tensor, or a tensor whose shape or dtype
disagrees with the cache geometry, must be turned into a ValueError before anything is
launched. Every call below fails in the wrapper, before the library is touched.
"""
import importlib

import pytest
import torch

_lib = importlib.import_module("nanokv-llm_amd._lib")
attn = importlib.import_module("nanokv-llm_amd.layers.attention")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")
rope = importlib.import_module("nanokv-llm_amd.layers.rotary_embedding")
meta = importlib.import_module("nanokv-llm_amd.engine.metadata")

BF = torch.bfloat16
I32 = torch.int32


def test_require_device():
    gpu = torch.device("cuda", 0)
    with pytest.raises(ValueError, match="expected GPU tensors"):
        _lib.require_device(torch.device("cpu"))
    with pytest.raises(ValueError, match="lens is on meta"):
        _lib.require_device(gpu, lens=torch.empty(2, device="meta"))
    _lib.require_device(gpu, lens=None)  # absent optional tensors are skipped
    with pytest.raises(ValueError, match="boom"):
        _lib.need(False, "boom")
    _lib.need(True, "unused")


def test_wrappers_reject_host_tensors():
    q = torch.zeros(2, 8, 128, dtype=BF)
    kc = torch.zeros(4, 16, 2, 128, dtype=BF)
    bt = torch.zeros(2, 4, dtype=I32)
    lens = torch.ones(2, dtype=I32)
    rows = torch.zeros(3, 2, 128, dtype=BF)
    with pytest.raises(ValueError, match="expected GPU"):
        attn.paged_decode(q, kc, kc, lens, bt, 0.1)
    with pytest.raises(ValueError, match="expected GPU"):
        attn.store_kvcache(rows, rows, kc, kc, torch.zeros(3, dtype=I32))
    cu_q = torch.tensor([0, 3], dtype=I32)
    with pytest.raises(ValueError, match="expected GPU"):
        attn.varlen_prefill(torch.zeros(3, 8, 128, dtype=BF), rows, rows, cu_q, cu_q, 3, 0.1)
    with pytest.raises(ValueError, match="expected GPU"):
        cu.compress_step(q, kc, kc, bt, lens, lens.clone(), torch.zeros(1, dtype=I32), 2, 17,
                         0.1)
    with pytest.raises(ValueError, match="expected GPU"):
        kvc.fp8_quantize(torch.zeros(16, dtype=BF))
    with pytest.raises(ValueError, match="expected GPU"):
        kvc.fp8_dequantize(torch.zeros(16, dtype=torch.uint8))
    with pytest.raises(ValueError, match="expected GPU"):
        rope.qk_norm_rope_store(torch.zeros(3, dtype=torch.int64), torch.zeros(3, 8, 128, dtype=BF),
                                rows, rows, torch.zeros(16, 1, 128))
    with pytest.raises(ValueError, match="expected GPU"):
        meta.build_step_metadata([0], [1], [[0]], 16, "cpu")
