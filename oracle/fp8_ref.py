"""ORACLE (test infrastructure): the fp8 (OCP E4M3FN) K/V format on the CPU.

Only tests, the smoke check and the bench's CPU baseline use this module; the
product path never imports it.

An fp8 pool (the K/V pool of nanokvllm/engine/model_runner.py:133-152 in one
byte per element) stores code = E4M3FN(clamp(x * (1/scale), -448, 448)), NaN
kept, round to nearest even, and reads code * scale; the store follows
store_kvcache (nanokvllm/layers/attention.py:10-40). torch's float8_e4m3fn
does the rounding; e4m3fn_table() and nearest_e4m3fn() restate the format from
its definition so the tests can pin torch's conversion.
"""
from __future__ import annotations

import torch

from .attention_ref import store_kvcache_ref

FP8_MAX = 448.0


def e4m3fn_table() -> torch.Tensor:
    """Value of each of the 256 codes from the OCP definition: sign, 4-bit exponent (bias 7),
    3-bit mantissa; exponent 0 is subnormal (m * 2^-9); S.1111.111 is NaN."""
    vals = []
    for c in range(256):
        s, e, m = c >> 7, (c >> 3) & 15, c & 7
        if e == 15 and m == 7:
            v = float("nan")
        elif e == 0:
            v = m * 2.0 ** -9
        else:
            v = (1 + m / 8) * 2.0 ** (e - 7)
        vals.append(-v if s else v)
    return torch.tensor(vals, dtype=torch.float64)


def nearest_e4m3fn(x: torch.Tensor) -> torch.Tensor:
    """Brute force: the code of the finite value nearest to each (finite, |x| <= 448) input:
    the magnitude rounds to the nearest of the 127 non-negative codes, ties to the even code
    (mantissa bit 0 clear), and the sign bit is the input's (so tiny negatives give -0)."""
    table = e4m3fn_table()
    cand = torch.arange(127)  # 0x00 .. 0x7E: +0 .. 448
    tv = table[cand]
    d = (x.double().abs().unsqueeze(-1) - tv).abs()
    best = d.min(dim=-1, keepdim=True).values
    tie = d == best
    key = torch.where(tie, 0, 2) + (cand & 1)  # nearest first, then the even code
    code = cand[torch.argmin(key, dim=-1)]
    neg = torch.signbit(x)
    return (code | (neg.long() << 7)).to(torch.uint8)


def fp8_quantize_ref(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """bf16 -> uint8 codes: E4M3FN(clamp(x * (1/scale), -448, 448)), NaN kept."""
    inv = 1.0 / torch.tensor(scale, dtype=torch.float32)  # fp32 division, as the kernels do
    y = x.float() * inv
    y = torch.where(torch.isnan(y), y, y.clamp(-FP8_MAX, FP8_MAX))
    return y.to(torch.float8_e4m3fn).view(torch.uint8)


def fp8_dequantize_ref(codes: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """uint8 codes -> bf16(value * scale)."""
    return (codes.view(torch.float8_e4m3fn).float() * scale).to(torch.bfloat16)


def store_kvcache_fp8_ref(key, value, k_cache, v_cache, slot_mapping, k_scale=1.0, v_scale=1.0):
    """store_kvcache into uint8 caches of codes (attention.py:21-40 with the fp8 format)."""
    store_kvcache_ref(fp8_quantize_ref(key, k_scale), fp8_quantize_ref(value, v_scale),
                      k_cache, v_cache, slot_mapping)
