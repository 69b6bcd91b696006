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


def test_attention_init_checks_kernel_limits():
    """Attention(...) rejects what the kernels would refuse at the first forward."""
    from types import SimpleNamespace
    off = SimpleNamespace(kv_compress_enabled=False)
    attn.Attention(32, 128, 0.1, 8, off, 2)
    attn.Attention(128, 128, 0.1, 1, off, 2)  # GQA group 128: one query per prefill tile
    with pytest.raises(ValueError, match="head_dim"):
        attn.Attention(32, 96, 0.1, 8, off, 2)
    with pytest.raises(ValueError, match="multiple of num_kv_heads"):
        attn.Attention(30, 128, 0.1, 8, off, 2)
    with pytest.raises(ValueError, match="GQA group"):
        attn.Attention(129, 128, 0.1, 1, off, 2)
    with pytest.raises(ValueError, match="GQA group"):
        attn.Attention(65, 256, 0.1, 1, off, 2)

    def cfg(W=4, kb=2, extra=1, agg=None):
        c = SimpleNamespace(kv_compress_enabled=True, kv_compress_window_blocks=W,
                            kv_compress_keep_blocks=kb, kv_compress_keep_extra_tokens=extra)
        if agg is not None:
            c.kv_compress_agg = agg
        return c

    attn.Attention(32, 128, 0.1, 8, cfg(), 2)
    with pytest.raises(ValueError, match="window_blocks"):
        attn.Attention(32, 128, 0.1, 8, cfg(W=65), 2)
    with pytest.raises(ValueError, match="kv_compress_agg"):
        attn.Attention(32, 128, 0.1, 8, cfg(agg="max"), 2)
    # cache geometry, checked once per binding at the first forward
    a = attn.Attention(32, 128, 0.1, 8, cfg(), 2)
    a.k_cache = torch.zeros(4, 256, 8, 128, dtype=BF)
    a._check_cache()
    a.k_cache = torch.zeros(4, 24, 8, 128, dtype=BF)
    with pytest.raises(ValueError, match="multiple of 16"):
        a._check_cache()
    a.k_cache = torch.zeros(4, 32, 8, 128, dtype=BF)  # window 128 tokens: block 32 not fused
    with pytest.raises(ValueError, match="multiple of 64"):
        a._check_cache()
    a.k_cache = torch.zeros(4, 256, 4, 128, dtype=BF)
    with pytest.raises(ValueError, match="k_cache must be"):
        a._check_cache()
    a = attn.Attention(32, 128, 0.1, 8, cfg(kb=0, extra=2), 2)
    a.k_cache = torch.zeros(4, 256, 8, 128, dtype=BF)
    with pytest.raises(ValueError, match="kept tokens"):
        a._check_cache()
    a = attn.Attention(32, 128, 0.1, 8, cfg(kb=4, extra=0), 2)  # keep == window: a no-op
    a.k_cache = torch.zeros(4, 256, 8, 128, dtype=BF)
    a._check_cache()


def test_shared_workspace_kept_only_when_captured(monkeypatch):
    """A regrown shared decode workspace is freed unless a graph capture saw it."""
    dev = torch.device("cpu")  # the bookkeeping only; no kernel runs
    monkeypatch.setattr(attn, "_SHARED_WS", {})
    monkeypatch.setattr(attn, "_CAPTURED_WS", set())
    monkeypatch.setattr(attn, "_RETIRED_WS", [])
    capturing = [False]
    monkeypatch.setattr(torch.cuda, "is_current_stream_capturing", lambda: capturing[0])
    w1 = attn.shared_decode_workspace(dev, 100)
    w2 = attn.shared_decode_workspace(dev, 1000)  # regrowth, w1 never captured: dropped
    assert w2.numel() >= 1000 and attn._RETIRED_WS == []
    capturing[0] = True
    assert attn.shared_decode_workspace(dev, 500) is w2  # used during a capture
    with pytest.raises(_lib.NkvError, match="before graph capture"):
        attn.shared_decode_workspace(dev, 10 ** 6)
    capturing[0] = False
    w3 = attn.shared_decode_workspace(dev, 10 ** 5)  # w2 is held by that graph: kept
    assert len(attn._RETIRED_WS) == 1 and attn._RETIRED_WS[0] is w2 and w3 is not w2
    assert attn.release_retired_decode_workspaces() == 1 and attn._RETIRED_WS == []
    del w1
