"""ORACLE (test infrastructure): q/k RMSNorm, rotary embedding and the fused
norm + rope + K/V store, on the CPU.

Only tests, the smoke check and the bench's CPU baseline use this module; the
product path never imports it.

Follows nanokvllm/layers/layernorm.py:16-26 (RMSNorm.rms_forward),
nanokvllm/layers/rotary_embedding.py:7-15 (apply_rotary_emb), :20-36 (the
cos|sin cache) and :38-49 (RotaryEmbedding.forward), composed as in
Qwen3Attention.forward, nanokvllm/models/qwen3.py:104-114, followed by the
store_kvcache call of Attention.forward (nanokvllm/layers/attention.py:71-73).
Every dtype conversion of the reference is kept: fp32 math, bf16 rounding
after the normalisation, after the weight multiply and after the rotation.
"""
from __future__ import annotations

import torch

from .attention_ref import store_kvcache_ref


def rotary_cos_sin_cache_ref(head_dim: int, max_position: int, base: float) -> torch.Tensor:
    """rotary_embedding.py:30-36: row p = [cos(p * inv_freq) | sin(p * inv_freq)], fp32.

    inv_freq[j] = 1 / base ** (2j / head_dim); returns [max_position, head_dim].
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, dtype=torch.float) / head_dim))
    t = torch.arange(max_position, dtype=torch.float)
    freqs = t[:, None] * inv_freq[None, :]
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def rms_norm_ref(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    """layernorm.py:21-26: bf16(bf16(x * rsqrt(mean(x^2) + eps)) * weight) over the last dim."""
    orig = x.dtype
    xf = x.float()
    var = xf.pow(2).mean(dim=-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return xf.to(orig) * weight


def apply_rotary_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """rotary_embedding.py:7-15: halves x1|x2 in fp32, [x1 c - x2 s | x2 c + x1 s] -> x.dtype."""
    x1, x2 = torch.chunk(x.float(), 2, dim=-1)
    y1 = x1 * cos - x2 * sin
    y2 = x2 * cos + x1 * sin
    return torch.cat((y1, y2), dim=-1).to(x.dtype)


def rotary_ref(positions, q, k, cos_sin_cache):
    """rotary_embedding.py:38-49 for q [N, Hq, D] and k [N, Hk, D] at int64 positions [N]."""
    cs = cos_sin_cache[positions.long()].unsqueeze(1)
    cos, sin = cs.chunk(2, dim=-1)
    return apply_rotary_ref(q, cos, sin), apply_rotary_ref(k, cos, sin)


def qk_norm_rope_store_ref(qkv, positions, q_norm_weight, k_norm_weight, eps, cos_sin_cache,
                           n_q_heads, n_kv_heads, head_dim=128, k_cache=None, v_cache=None,
                           slot_mapping=None):
    """qwen3.py:104-114 up to the attention call, then attention.py:71-73's store.

    qkv [N, (Hq + 2 Hk) * D] bf16. Norm weights None = no q/k norm (the
    qkv_bias=True branch). Returns (q, k, v) as [N, H, D]; when the caches are
    given, row slot_mapping[i] receives k[i] / v[i] (slot -1 skipped).
    """
    N = qkv.size(0)
    qs, ks = n_q_heads * head_dim, n_kv_heads * head_dim
    q, k, v = qkv.split([qs, ks, ks], dim=-1)
    q = q.reshape(N, n_q_heads, head_dim)
    k = k.reshape(N, n_kv_heads, head_dim)
    v = v.reshape(N, n_kv_heads, head_dim)
    if q_norm_weight is not None:
        q = rms_norm_ref(q, q_norm_weight, eps)
        k = rms_norm_ref(k, k_norm_weight, eps)
    q, k = rotary_ref(positions, q, k, cos_sin_cache)
    if k_cache is not None:
        store_kvcache_ref(k, v, k_cache, v_cache, slot_mapping)
    return q, k, v
