"""Paged decode on the GPU vs the fp32 oracle: max abs err <= 2e-2 (bf16 output)."""
import importlib

import pytest
import torch

from oracle.attention_ref import paged_decode_ref, store_kvcache_ref

pytestmark = pytest.mark.gpu
TOL = 2e-2
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")


def _check(nkv, dev, q, kc, vc, ctx, bt, scale, kc_gpu=None, vc_gpu=None):
    kg = kc.to(dev) if kc_gpu is None else kc_gpu
    vg = vc.to(dev) if vc_gpu is None else vc_gpu
    out = nkv.paged_decode(q.to(dev), kg, vg, ctx.to(dev), bt.to(dev), scale)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.float(), kc, vc, ctx, bt, scale)
    err = (out.float().cpu() - ref).abs().max().item()
    assert err <= TOL, f"max abs err {err}"
    return out


def test_decode_qwen3_0_6b_with_store(nkv, dev):
    wl = wl_mod.decode_qwen3_0_6b(seed=1)
    kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    bt, slots = wl["block_tables"][0], wl["slot_mappings"][0]
    kg, vg = kc.to(dev), vc.to(dev)
    nkv.store_kvcache(wl["key"].to(dev), wl["value"].to(dev), kg, vg, slots.to(dev))
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, slots)
    out = _check(nkv, dev, wl["q"], kc, vc, wl["context_lens"], bt, wl["scale"], kg, vg)
    assert out.shape == (4, 16, 128)


@pytest.mark.parametrize("Hq,Hk", [(32, 8), (64, 8), (8, 8), (16, 8), (128, 8)])
def test_decode_qwen3_8b_shapes(nkv, dev, Hq, Hk):
    wl = wl_mod.decode_workload(6, Hq, Hk, 2048, 8192, 6 * 32 + 4, seed=2)
    _check(nkv, dev, wl["q"], wl["k_cache"], wl["v_cache"], wl["context_lens"],
           wl["block_tables"][0], wl["scale"])


def test_decode_edge_lengths(nkv, dev):
    g = torch.Generator().manual_seed(21)
    nb, B, Hk, D = 12, 256, 8, 128
    kc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    ctx = torch.tensor([0, 1, 255, 256, 257, 511, 512, 513], dtype=torch.int32)
    bt = torch.full((8, 3), -1, dtype=torch.int32)
    ids = torch.randperm(nb, generator=g).tolist()  # exactly 12 blocks are needed
    p = 0
    for i, n in enumerate(ctx.tolist()):
        k = (n + B - 1) // B
        bt[i, :k] = torch.tensor(ids[p:p + k], dtype=torch.int32)
        p += k
    q = torch.randn(8, 32, D, generator=g).to(torch.bfloat16)
    out = _check(nkv, dev, q, kc, vc, ctx, bt, D ** -0.5)
    assert torch.all(out[0] == 0)  # empty context -> zeros
    # ctx = 1 -> exactly the first value row (softmax weight 1)
    assert torch.equal(out[1, :4].cpu(), vc[int(bt[1, 0]), 0, 0].expand(4, D))


def test_decode_strided_q_and_graph_padding(nkv, dev):
    wl = wl_mod.decode_workload(5, 32, 8, 300, 1500, 40, seed=3)
    bt = wl["block_tables"][0]
    bt0 = torch.where(bt < 0, torch.zeros_like(bt), bt)  # graph buffers pad with 0
    bt0 = torch.cat([bt0, torch.zeros(5, 3, dtype=torch.int32)], dim=1)  # wider table
    qkv = torch.randn(5, 48 * 128).to(torch.bfloat16)
    q = qkv[:, :32 * 128].view(5, 32, 128)  # row stride 48*128
    qg = qkv.to(dev)[:, :32 * 128].view(5, 32, 128)
    kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    out = nkv.paged_decode(qg, kg, vg, wl["context_lens"].to(dev), bt0.to(dev), wl["scale"])
    ref = paged_decode_ref(q.float(), wl["k_cache"], wl["v_cache"], wl["context_lens"], bt,
                           wl["scale"])
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


def test_decode_block_permutation_invariance(nkv, dev):
    wl = wl_mod.decode_workload(4, 32, 8, 600, 2000, 40, seed=4)
    kc, vc, bt = wl["k_cache"], wl["v_cache"], wl["block_tables"][0]
    perm = torch.randperm(40, generator=torch.Generator().manual_seed(5))
    inv = torch.argsort(perm)
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].to(torch.int32), bt)
    a = nkv.paged_decode(wl["q"].to(dev), kc.to(dev), vc.to(dev), wl["context_lens"].to(dev),
                         bt.to(dev), wl["scale"])
    b = nkv.paged_decode(wl["q"].to(dev), kc[perm].to(dev), vc[perm].to(dev),
                         wl["context_lens"].to(dev), bt2.to(dev), wl["scale"])
    assert torch.equal(a, b)  # same bytes in the same order -> bitwise identical


def test_decode_attention_module(nkv, dev):
    """Attention.forward on the decode branch: store, then attend (attention.py:67-108)."""
    from types import SimpleNamespace
    wl = wl_mod.decode_qwen3_0_6b(seed=6)
    cfg = SimpleNamespace(kv_compress_enabled=False)
    attn = nkv.Attention(16, 128, 128 ** -0.5, 8, cfg, 1)
    attn.k_cache, attn.v_cache = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    bt, slots = wl["block_tables"][0], wl["slot_mappings"][0]
    nkv.set_context(True, slot_mapping=slots.to(dev), context_lens=wl["context_lens"].to(dev),
                    block_tables=bt.to(dev))
    o = attn(wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev), 0)
    nkv.reset_context()
    kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, slots)
    ref = paged_decode_ref(wl["q"].float(), kc, vc, wl["context_lens"], bt, wl["scale"])
    assert o.shape == (4, 1, 16, 128)
    assert (o[:, 0].float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("seed", [0, 1])
def test_decode_ragged_batch_over_64(nkv, dev, seed):
    """200 sequences (several 64-sequence cursor batches), lengths 0..700 with many
    short ones: every wave crosses many (sequence, KV head) segments."""
    g = torch.Generator().manual_seed(100 + seed)
    bs, Hq, Hk, D, B = 200, 32, 8, 128, 256
    ctx = torch.randint(0, 700, (bs,), generator=g, dtype=torch.int32)
    ctx[::7] = torch.randint(1, 20, (len(ctx[::7]),), generator=g, dtype=torch.int32)
    ctx[5] = 0
    ctx[64] = 0
    ctx[199] = 0
    need = [(int(c) + B - 1) // B for c in ctx]
    nb = sum(need) + 3
    perm = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((bs, 3), -1, dtype=torch.int32)
    p = 0
    for i, n in enumerate(need):
        bt[i, :n] = torch.tensor(perm[p:p + n], dtype=torch.int32)
        p += n
    kc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(bs, Hq, D, generator=g).to(torch.bfloat16)
    out = _check(nkv, dev, q, kc, vc, ctx, bt, D ** -0.5)
    assert torch.all(out[ctx == 0] == 0)


def test_decode_qwen3_32b_long_context(nkv, dev):
    """Qwen3-32B geometry (Hq 64, Hk 8: GQA group 8), contexts log-uniform up to 16384
    (64 blocks per sequence, the block-id window's full width), some already compressed."""
    wl = wl_mod.decode_qwen3_32b_longctx(seed=6, bs=8, n_blocks=400)
    kc, vc = wl["k_cache"], wl["v_cache"]
    bt, slots = wl["block_tables"][0], wl["slot_mappings"][0]
    kg, vg = kc.to(dev), vc.to(dev)
    nkv.store_kvcache(wl["key"].to(dev), wl["value"].to(dev), kg, vg, slots.to(dev))
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, slots)
    _check(nkv, dev, wl["q"], kc, vc, wl["context_lens"], bt, wl["scale"], kg, vg)
    assert bool(wl["compressed"].any())


def test_decode_64_block_window_boundary(nkv, dev):
    """Contexts of 64*256 +- a few tokens: the block-id window reloads after 64 blocks."""
    g = torch.Generator().manual_seed(31)
    Hq, Hk, D, B = 32, 8, 128, 256
    ctx = torch.tensor([64 * B - 1, 64 * B, 64 * B + 1, 70 * B + 5], dtype=torch.int32)
    need = [(int(c) + B - 1) // B for c in ctx]
    nb = sum(need) + 2
    perm = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((4, max(need)), -1, dtype=torch.int32)
    p = 0
    for i, n in enumerate(need):
        bt[i, :n] = torch.tensor(perm[p:p + n], dtype=torch.int32)
        p += n
    kc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(4, Hq, D, generator=g).to(torch.bfloat16)
    _check(nkv, dev, q, kc, vc, ctx, bt, D ** -0.5)


@pytest.mark.parametrize("Hq,Hk", [(32, 8), (16, 2)])
def test_decode_one_long_sequence_many_partials(nkv, dev, Hq, Hk):
    """One 30k-token sequence: its chunk stream is split over ~120 waves per head group, so
    the combine merges more than 64 partials per query head (two per lane)."""
    wl = wl_mod.decode_workload(1, Hq, Hk, 29000, 30500, 130, seed=8)
    _check(nkv, dev, wl["q"], wl["k_cache"], wl["v_cache"], wl["context_lens"],
           wl["block_tables"][0], wl["scale"])
