"""Paged decode with two KV heads per wave.

That path is taken when Hk is even, 2G <= 16 and the block table is wide enough for the
work to fill every resident wave (batch x table width x B/16 x Hk >= 32 x resident waves).
A wide table forces it here even with small, ragged contexts; the same rows in a narrow
table take the one-head path. fp8 caches take four KV heads per wave instead of two when
Hk % 4 == 0 and 4G <= 16. Checks: both paths against the fp32 oracle (2e-2), the two paths
against each other (1e-2: only the split points of the chunk stream differ), the fp8
kernel (scales 1) against the bf16 kernel over the dequantized cache, bit for bit on the
same head grouping, and the four-head fp8 path against the oracle over dequantized values.
"""
import importlib
import random

import pytest
import torch

from oracle.attention_ref import paged_decode_ref

pytestmark = pytest.mark.gpu
TOL = 2e-2
D = 128
kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")


def _state(seed, bs, Hq, Hk, B, top):
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    lens = [rng.choice([0, 1, rng.randrange(1, top + 1), rng.randrange(1, top + 1)])
            for _ in range(bs)]
    need = [(n + B - 1) // B for n in lens]
    narrow = max(1, max(need))
    # wide enough for the pair path on a 256-CU part with 8 resident waves per CU
    wide = max(narrow, -(-(32 * 2048 * 2) // (bs * (B // 16) * Hk)))
    n_blocks = sum(need) + 3
    free = list(range(n_blocks))
    rng.shuffle(free)
    rows = [[free.pop() for _ in range(k)] for k in need]
    pad = rng.choice([-1, 0])
    bt_n = torch.tensor([r + [pad] * (narrow - len(r)) for r in rows], dtype=torch.int32)
    bt_w = torch.tensor([r + [pad] * (wide - len(r)) for r in rows], dtype=torch.int32)
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(bs, Hq, D, generator=g).to(torch.bfloat16)
    return q, kc, vc, torch.tensor(lens, dtype=torch.int32), bt_n, bt_w


@pytest.mark.parametrize("Hq,Hk,B", [(2, 2, 256), (8, 2, 256), (16, 4, 256), (32, 8, 256),
                                     (64, 8, 256), (8, 8, 256), (16, 8, 16), (128, 8, 256)])
def test_pair_and_single_paths_vs_oracle(nkv, dev, Hq, Hk, B):
    q, kc, vc, ctx, bt_n, bt_w = _state(Hq * 7 + Hk + B, 17, Hq, Hk, B, 3000)
    args = (q.to(dev), kc.to(dev), vc.to(dev), ctx.to(dev))
    wide = nkv.paged_decode(*args, bt_w.to(dev), D ** -0.5)
    narrow = nkv.paged_decode(*args, bt_n.to(dev), D ** -0.5)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.float(), kc, vc, ctx, bt_n, D ** -0.5)
    assert (wide.float().cpu() - ref).abs().max().item() <= TOL
    assert (narrow.float().cpu() - ref).abs().max().item() <= TOL
    assert (wide.float() - narrow.float()).abs().max().item() <= 1e-2


@pytest.mark.parametrize("Hq,Hk", [(32, 8), (16, 2), (8, 8), (32, 16)])
def test_pair_path_fp8_equals_bf16_over_dequantized(nkv, dev, Hq, Hk):
    q, kc, vc, ctx, _, bt_w = _state(50 + Hq + Hk, 12, Hq, Hk, 256, 4000)
    kq, vq = kvc.fp8_quantize(kc.to(dev)), kvc.fp8_quantize(vc.to(dev))
    kd, vd = kvc.fp8_dequantize(kq), kvc.fp8_dequantize(vq)
    args = (ctx.to(dev), bt_w.to(dev), D ** -0.5)
    a = nkv.paged_decode(q.to(dev), kq, vq, *args)
    b = nkv.paged_decode(q.to(dev), kd, vd, *args)
    if Hk % 4 == 0 and Hq // Hk <= 4:  # fp8: four heads per wave, bf16: two
        assert (a.float() - b.float()).abs().max().item() <= 1e-2
    else:
        assert torch.equal(a, b)


@pytest.mark.parametrize("Hq,Hk,B", [(8, 8, 256), (16, 8, 256), (32, 8, 256), (4, 4, 256),
                                     (16, 4, 64), (32, 16, 16)])
def test_four_head_fp8_path_vs_oracle(nkv, dev, Hq, Hk, B):
    q, kc, vc, ctx, bt_n, bt_w = _state(90 + Hq + Hk + B, 15, Hq, Hk, B, 3500)
    kq, vq = kvc.fp8_quantize(kc.to(dev)), kvc.fp8_quantize(vc.to(dev))
    kd, vd = kvc.fp8_dequantize(kq).cpu(), kvc.fp8_dequantize(vq).cpu()
    out = nkv.paged_decode(q.to(dev), kq, vq, ctx.to(dev), bt_w.to(dev), D ** -0.5)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.float(), kd, vd, ctx, bt_n, D ** -0.5)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


def test_four_head_fp8_big_batch_and_window_reload(nkv, dev):
    """Four-head fp8 path over 130 sequences (three 64-sequence cursor batches): mostly short
    or empty contexts, plus four past 64 blocks, so the 64-entry block-id window reloads."""
    rng = random.Random(77)
    g = torch.Generator().manual_seed(77)
    bs, Hq, Hk, B = 130, 32, 8, 256
    lens = [rng.choice([0, 1, rng.randrange(1, 600), rng.randrange(1, 600)]) for _ in range(bs)]
    for i in (3, 64, 100, 129):
        lens[i] = 64 * B + rng.randrange(-3, 2 * B)
    need = [(n + B - 1) // B for n in lens]
    width = max(need)
    n_blocks = sum(need) + 3
    free = list(range(n_blocks))
    rng.shuffle(free)
    bt = torch.tensor([[free.pop() for _ in range(k)] + [-1] * (width - k) for k in need],
                      dtype=torch.int32)
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(bs, Hq, D, generator=g).to(torch.bfloat16)
    ctx = torch.tensor(lens, dtype=torch.int32)
    kq, vq = kvc.fp8_quantize(kc.to(dev)), kvc.fp8_quantize(vc.to(dev))
    out = nkv.paged_decode(q.to(dev), kq, vq, ctx.to(dev), bt.to(dev), D ** -0.5)
    torch.cuda.synchronize()
    kd, vd = kvc.fp8_dequantize(kq).cpu(), kvc.fp8_dequantize(vq).cpu()
    ref = paged_decode_ref(q.float(), kd, vd, ctx, bt, D ** -0.5)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL
    assert torch.all(out[ctx.to(dev) == 0] == 0)
