"""Rotary embedding and the fused q/k RMSNorm + RoPE + K/V store.

Mirrors nanokvllm/layers/rotary_embedding.py (``RotaryEmbedding`` with the
same constructor, ``cos_sin_cache`` buffer and ``forward(positions, query,
key)``; ``get_rope``) and adds ``qk_norm_rope_store``, which does the work of
Qwen3Attention.forward between the qkv projection and the attention call
(nanokvllm/models/qwen3.py:104-113: q_norm/k_norm, rotary_emb) together with
the store_kvcache call at the top of Attention.forward
(nanokvllm/layers/attention.py:71-73) in one kernel. All compute runs in
libnkv_amd.so on the caller's current stream.
"""
from __future__ import annotations

from functools import lru_cache

import torch
from torch import nn

from .. import _lib

_BF16 = torch.bfloat16


def _rows(x: torch.Tensor, heads: int, head_dim: int, dtype=_BF16):
    assert x.dtype == dtype and x.dim() == 3 and x.size(1) == heads and x.size(2) == head_dim
    assert x.stride(2) == 1 and x.stride(1) == head_dim, "heads must be contiguous in a row"
    return x.data_ptr(), x.stride(0)


def qk_norm_rope_store(positions: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                       v: torch.Tensor | None, cos_sin_cache: torch.Tensor,
                       q_norm_weight: torch.Tensor | None = None,
                       k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, need_k: bool = True,
                       q_out: torch.Tensor | None = None):
    """q [N, Hq, D], k/v [N, Hk, D] (row-strided views of the qkv output) ->
    (q', k' or None, v).

    q' = rope(norm(q)), k' = rope(norm(k)) with the reference's roundings
    (layernorm.py:21-26, rotary_embedding.py:7-15); norm is skipped when the
    weights are None (the qkv_bias=True branch of qwen3.py:109). With caches,
    k' and v are written to row slot_mapping[i] (slot -1 skipped) as
    store_kvcache does. ``need_k=False`` skips the contiguous k' output (when
    attention reads K back from the cache). v is returned unchanged. q, k, v, the
    norm weights, the outputs and the caches share one dtype, bf16 or fp16 (the
    roundings are then to fp16).
    """
    N, Hq, D = q.shape
    Hk = k.size(1)
    _lib.require_device(q.device, k=k, v=v, positions=positions, cos_sin_cache=cos_sin_cache,
                        q_norm_weight=q_norm_weight, k_norm_weight=k_norm_weight,
                        k_cache=k_cache, v_cache=v_cache, slot_mapping=slot_mapping, q_out=q_out)
    dt = q.dtype
    f16 = _lib.is_f16(q, "qk_norm_rope_store: q")
    q_ptr, q_rs = _rows(q, Hq, D, dt)
    k_ptr, k_rs = _rows(k, Hk, D, dt)
    assert k.size(0) == N and positions.dtype == torch.int64 and positions.is_contiguous()
    assert positions.numel() == N
    cs = cos_sin_cache.reshape(cos_sin_cache.size(0), -1)
    assert cs.dtype == torch.float32 and cs.is_contiguous() and cs.size(1) == D
    if (q_norm_weight is None) != (k_norm_weight is None):
        raise ValueError("give both q/k norm weights or neither")
    if q_norm_weight is not None:
        assert q_norm_weight.dtype == dt and k_norm_weight.dtype == dt
        assert q_norm_weight.is_contiguous() and k_norm_weight.is_contiguous()
        assert q_norm_weight.numel() == D and k_norm_weight.numel() == D
    if q_out is None:
        q_out = torch.empty(N, Hq, D, dtype=dt, device=q.device)
    _rows(q_out, Hq, D, dt)
    _lib.need(q_out.size(0) == N, "qk_norm_rope_store: q_out needs one row per token")
    store = k_cache is not None and k_cache.numel() > 0
    k_out = torch.empty(N, Hk, D, dtype=dt, device=q.device) if (need_k or not store) else None
    v_ptr, v_rs = (0, 0)
    n_slots = 0
    if store:
        assert v is not None and slot_mapping is not None
        v_ptr, v_rs = _rows(v, Hk, D, dt)
        _lib.need(v.size(0) == N, "qk_norm_rope_store: v needs one row per token")
        assert k_cache.dtype == dt and v_cache.dtype == dt
        assert k_cache.is_contiguous() and v_cache.is_contiguous()
        assert k_cache.size(-1) == D and k_cache.size(-2) == Hk and v_cache.shape == k_cache.shape
        assert slot_mapping.dtype == torch.int32 and slot_mapping.is_contiguous()
        assert slot_mapping.numel() == N
        n_slots = k_cache.numel() // (Hk * D)
    fn = _lib.lib().nkv_qk_norm_rope_store_f16 if f16 else _lib.lib().nkv_qk_norm_rope_store
    rc = fn(
        q_ptr, q_rs, k_ptr, k_rs, v_ptr or None, v_rs, positions.data_ptr(),
        q_norm_weight.data_ptr() if q_norm_weight is not None else None,
        k_norm_weight.data_ptr() if k_norm_weight is not None else None, float(eps),
        cs.data_ptr(), cs.size(0), q_out.data_ptr(), q_out.stride(0),
        k_out.data_ptr() if k_out is not None else None,
        k_cache.data_ptr() if store else None, v_cache.data_ptr() if store else None,
        slot_mapping.data_ptr() if store else None, n_slots, N, Hq, Hk, D, _lib.stream_of(q))
    _lib.check(rc, "qk_norm_rope_store")
    return q_out, k_out, v


class RotaryEmbedding(nn.Module):
    """rotary_embedding.py:18-49: cos|sin table [max_pos, 1, rotary_dim] (fp32) and
    forward(positions, query, key) -> (rope(query), rope(key)) in one launch.

    The table is computed once on the host in fp32 and then moved to ``device``:
    a device pow() one ulp away from the host's shifts inv_freq, and at positions
    near 4e4 that moves the angle by ~2e-3 rad, so a table built on the device
    would depend on its math library.
    """

    def __init__(self, head_size: int, rotary_dim: int, max_position_embeddings: int,
                 base: float, device=None) -> None:
        super().__init__()
        self.head_size = head_size
        assert rotary_dim == head_size
        inv_freq = 1.0 / (base ** (torch.arange(0, rotary_dim, 2, dtype=torch.float,
                                                device="cpu") / rotary_dim))
        t = torch.arange(max_position_embeddings, dtype=torch.float, device="cpu")
        freqs = t[:, None] * inv_freq[None, :]
        cache = torch.cat((freqs.cos(), freqs.sin()), dim=-1).unsqueeze_(1)
        self.register_buffer("cos_sin_cache", cache.to(device) if device else cache,
                             persistent=False)

    def forward(self, positions: torch.Tensor, query: torch.Tensor, key: torch.Tensor):
        D = self.head_size
        q = query.view(query.size(0), -1, D) if query.dim() == 2 else query
        k = key.view(key.size(0), -1, D) if key.dim() == 2 else key
        qo, ko, _ = qk_norm_rope_store(positions, q, k, None, self.cos_sin_cache)
        return qo.view(query.shape), ko.view(key.shape)


@lru_cache(maxsize=8)
def _get_rope_cached(head_size, rotary_dim, max_position, base, device):
    return RotaryEmbedding(head_size, rotary_dim, max_position, base, device=device)


def get_rope(head_size: int, rotary_dim: int, max_position: int, base: float,
             rope_scaling: dict | None = None, device=None):
    """rotary_embedding.py:73-85: only the default rope type is supported."""
    if isinstance(rope_scaling, dict):
        if rope_scaling.get("rope_type", "default") != "default":
            raise NotImplementedError(f"unsupported rope_scaling: {rope_scaling}")
        rope_scaling = None
    assert rope_scaling is None
    return _get_rope_cached(head_size, rotary_dim, max_position, base,
                            None if device is None else str(device))
