"""The paged K/V pool and its fp8 (OCP E4M3FN) option.

``KVCachePool`` mirrors ModelRunner.allocate_kv_cache
(nanokvllm/engine/model_runner.py:133-152): one [2, layers, blocks, block_size,
Hk, D] tensor sized from the free device memory as the reference does
(total * gpu_memory_utilization - used - peak + current, divided by the bytes
of one block across layers), whose per-layer views are handed to every module
that has ``k_cache``/``v_cache`` attributes. With ``dtype=torch.float8_e4m3fn``
a block takes half the bytes (twice the cached tokens in the same HBM); the
layers then store E4M3FN(clamp(x / scale)) and attention reads code * scale,
with one scale per K and V cache (``k_scale``/``v_scale`` on each module).
"""
from __future__ import annotations

import torch

from .. import _lib

FP8 = torch.float8_e4m3fn


def is_fp8(t: torch.Tensor) -> bool:
    return t.dtype == FP8


def fp8_quantize(x: torch.Tensor, scale: float = 1.0, out: torch.Tensor | None = None):
    """bf16 -> E4M3FN codes of clamp(x * (1/scale), -448, 448) (NaN kept)."""
    assert x.dtype == torch.bfloat16 and x.is_contiguous() and x.numel() % 16 == 0
    _lib.require_device(x.device, out=out)
    if out is None:
        out = torch.empty(x.shape, dtype=FP8, device=x.device)
    _lib.need(out.element_size() == 1 and out.is_contiguous() and out.numel() == x.numel(),
              "fp8_quantize: out must be contiguous 1-byte codes, one per element")
    rc = _lib.lib().nkv_fp8_quantize(x.data_ptr(), x.numel(), float(scale), out.data_ptr(),
                                     _lib.stream_of(x))
    _lib.check(rc, "fp8_quantize")
    return out


def fp8_dequantize(codes: torch.Tensor, scale: float = 1.0, out: torch.Tensor | None = None):
    """E4M3FN codes -> bf16(value * scale)."""
    assert codes.element_size() == 1 and codes.is_contiguous() and codes.numel() % 16 == 0
    _lib.require_device(codes.device, out=out)
    if out is None:
        out = torch.empty(codes.shape, dtype=torch.bfloat16, device=codes.device)
    _lib.need(out.dtype == torch.bfloat16 and out.is_contiguous() and out.numel() == codes.numel(),
              "fp8_dequantize: out must be contiguous bf16, one per code")
    rc = _lib.lib().nkv_fp8_dequantize(codes.data_ptr(), codes.numel(), float(scale),
                                       out.data_ptr(), _lib.stream_of(codes))
    _lib.check(rc, "fp8_dequantize")
    return out


class KVCachePool:
    """One K/V tensor for every layer (model_runner.py:133-152): bf16 or fp16 (the model's
    dtype, as the reference allocates it) or fp8."""

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, block_size: int = 256,
                 dtype: torch.dtype = torch.bfloat16, gpu_memory_utilization: float = 0.8,
                 num_blocks: int | None = None, device="cuda", k_scale: float = 1.0,
                 v_scale: float = 1.0):
        if dtype not in (torch.bfloat16, torch.float16, FP8):
            raise ValueError("the pool holds bf16, fp16 or float8_e4m3fn")
        self.block_size, self.dtype = block_size, dtype
        itemsize = torch.tensor([], dtype=dtype).element_size()
        self.block_bytes = 2 * num_layers * block_size * num_kv_heads * head_dim * itemsize
        if num_blocks is None:
            free, total = torch.cuda.mem_get_info(device)
            stats = torch.cuda.memory_stats(device)
            used = total - free
            peak = stats.get("allocated_bytes.all.peak", 0)
            current = stats.get("allocated_bytes.all.current", 0)
            num_blocks = int(total * gpu_memory_utilization - used - peak + current) \
                // self.block_bytes
        if num_blocks <= 0:
            raise RuntimeError("no device memory left for the K/V pool")
        self.num_blocks = num_blocks
        self.kv_cache = torch.empty(2, num_layers, num_blocks, block_size, num_kv_heads,
                                    head_dim, dtype=dtype, device=device)
        self.k_scale, self.v_scale = float(k_scale), float(v_scale)

    def bind(self, modules) -> int:
        """Assign layer i's views to the i-th module with k_cache/v_cache (model_runner.py
        :148-152); returns the number of layers bound."""
        layer = 0
        for m in modules:
            if hasattr(m, "k_cache") and hasattr(m, "v_cache"):
                m.k_cache = self.kv_cache[0, layer]
                m.v_cache = self.kv_cache[1, layer]
                m.k_scale, m.v_scale = self.k_scale, self.v_scale
                layer += 1
        return layer
