"""GQA groups outside the powers of two and above 16: decode, prefill and the compression
step against the oracle for g = 3, 5, 6, 7, 16, 17, 20, 32, 64, 128 (decode splits a group
above 16 over waves of 16 query heads; prefill tiles hold 128 query x head rows; the
compression step scores such groups in passes of 16), and Qwen3-14B geometry (40 query
heads over 8 KV heads, g = 5) through Attention.forward.

The reference hands any Hq % Hk == 0 to flash-attn (nanokvllm/layers/attention.py:96-107)
with head counts from the model config (nanokvllm/models/qwen3.py:53-60). Bars as in the rest
of the suite: bf16 attention outputs within 2e-2 of the fp32 oracle; importance within rtol
1e-4; kept sets exact given the scores; compaction and lengths bit-exact.
"""
import importlib
import random
from types import SimpleNamespace

import pytest
import torch

from oracle.attention_ref import paged_decode_ref, store_kvcache_ref, varlen_prefill_ref
from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)

pytestmark = pytest.mark.gpu
TOL = 2e-2
D = 128
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")


def _randn(shape, g):
    return torch.randn(shape, generator=g).to(torch.bfloat16)


def _tables(rng, lens, B, n_blocks, width, pad=-1):
    free = list(range(n_blocks))
    rng.shuffle(free)
    rows = []
    for n in lens:
        nb = (n + B - 1) // B
        rows.append([free.pop() for _ in range(nb)] + [pad] * (width - nb))
    return torch.tensor(rows, dtype=torch.int32).reshape(len(lens), width)


@pytest.mark.parametrize("Hq,Hk", [(24, 8), (40, 8), (48, 8), (56, 8), (128, 8), (12, 4),
                                   (10, 2), (7, 1), (16, 1), (17, 1), (40, 2), (64, 2), (64, 1),
                                   (128, 1)])
def test_decode_gqa_groups(nkv, dev, Hq, Hk):
    """Table widths both below and above the two-heads-per-wave threshold."""
    for width_blocks, bs, hi in ((4, 9, 1000), (32, 24, 8000)):
        wl = wl_mod.decode_workload(bs, Hq, Hk, 1, hi, bs * width_blocks + 8,
                                    seed=Hq * 100 + Hk + width_blocks)
        print(f"decode Hq={Hq} Hk={Hk} bs={bs} max_ctx={hi}", flush=True)
        bt = wl["block_tables"][0]
        out = nkv.paged_decode(wl["q"].to(dev), wl["k_cache"].to(dev), wl["v_cache"].to(dev),
                               wl["context_lens"].to(dev), bt.to(dev), wl["scale"])
        torch.cuda.synchronize()
        ref = paged_decode_ref(wl["q"].float(), wl["k_cache"], wl["v_cache"],
                               wl["context_lens"], bt, wl["scale"])
        assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("Hq,Hk", [(24, 8), (40, 8), (48, 8), (56, 8), (128, 8), (10, 2),
                                   (40, 2), (64, 2), (64, 1), (128, 1)])
@pytest.mark.parametrize("paged", [True, False])
def test_prefill_gqa_groups(nkv, dev, Hq, Hk, paged):
    rng = random.Random(Hq * 7 + Hk + int(paged))
    g = torch.Generator().manual_seed(Hq * 7 + Hk + int(paged))
    B = 64
    Lq = [1, 37, 300, 129]
    Lk = [1 + 5, 37, 300 + 400, 129 + 64]
    cq = torch.tensor([0] + torch.tensor(Lq).cumsum(0).tolist(), dtype=torch.int32)
    ck = torch.tensor([0] + torch.tensor(Lk).cumsum(0).tolist(), dtype=torch.int32)
    q = _randn((int(cq[-1]), Hq, D), g)
    print(f"prefill Hq={Hq} Hk={Hk} paged={paged}", flush=True)
    if paged:
        n_blocks = sum((k + B - 1) // B for k in Lk) + 3
        bt = _tables(rng, Lk, B, n_blocks, max((k + B - 1) // B for k in Lk))
        kc, vc = _randn((n_blocks, B, Hk, D), g), _randn((n_blocks, B, Hk, D), g)
        out = nkv.varlen_prefill(q.to(dev), kc.to(dev), vc.to(dev), cq.to(dev), ck.to(dev),
                                 max(Lq), D ** -0.5, block_tables=bt.to(dev))
        ref = varlen_prefill_ref(q.float(), kc, vc, cq, ck, D ** -0.5, block_tables=bt)
    else:
        k, v = _randn((int(ck[-1]), Hk, D), g), _randn((int(ck[-1]), Hk, D), g)
        out = nkv.varlen_prefill(q.to(dev), k.to(dev), v.to(dev), cq.to(dev), ck.to(dev),
                                 max(Lq), D ** -0.5)
        ref = varlen_prefill_ref(q.float(), k, v, cq, ck, D ** -0.5)
    torch.cuda.synchronize()
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("Hq,Hk", [(24, 8), (40, 8), (48, 8), (56, 8), (64, 8), (128, 8),
                                   (64, 2), (40, 2)])
@pytest.mark.parametrize("agg", ["all", "group"])
def test_compress_step_gqa_groups(nkv, dev, Hq, Hk, agg):
    wl = wl_mod.compress_workload(40, Hq, Hk, 1500, 4096, 6, seed=Hq + Hk, selected_only=True)
    bt, base = wl["block_tables"], wl["context_lens"]
    sel = wl["seq_idx"]
    print(f"compress Hq={Hq} Hk={Hk} agg={agg} sel={sel}", flush=True)
    kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    ctx = base.clone().to(dev)
    keep, imp = cu.compress_step(wl["q"].to(dev), kg, vg, bt.to(dev), base.to(dev), ctx,
                                 torch.tensor(sel, dtype=torch.int32, device=dev), 4, 513,
                                 D ** -0.5, agg)
    torch.cuda.synchronize()
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt, base, st, 256, 4)
    k_sub, _ = gather_kv_by_slots_ref(wl["k_cache"], wl["v_cache"], slots)
    ref_imp = snapkv_importance_ref(wl["q"].index_select(0, st).unsqueeze(2), k_sub, 1, "fp32",
                                    agg)
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    assert torch.equal(keep.cpu()[..., 1:-1].long(), select_topk_ref(imp.cpu(), 511))
    kc, vc, ctx_ref = wl["k_cache"].clone(), wl["v_cache"].clone(), base.clone()
    compress_compact_ref(None, kc, vc, bt, base, ctx_ref, sel, 256, 4, 2, 1, 0, 1,
                         keep_idx=keep.cpu().long())
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    assert torch.equal(ctx.cpu(), ctx_ref)


def test_attention_qwen3_14b_geometry(nkv, dev):
    """Attention(40, 128, scale, 8): a prefill step, then a decode step with a compression
    step (agg "all", the reference) on the last layer of two, through Attention.forward."""
    g = torch.Generator().manual_seed(14)
    Hq, Hk, B, L = 40, 8, 256, 2
    cfg = SimpleNamespace(kv_compress_enabled=True, kv_compress_window_blocks=4,
                          kv_compress_keep_blocks=2, kv_compress_keep_extra_tokens=1)
    layers = [nkv.Attention(Hq, D, D ** -0.5, Hk, cfg, L) for _ in range(L)]
    lens = [1300, 2100, 1030]
    n_blocks = 40
    rng = random.Random(14)
    bt = _tables(rng, [n + 1 for n in lens], B, n_blocks, 12)
    caches = [(_randn((n_blocks, B, Hk, D), g), _randn((n_blocks, B, Hk, D), g))
              for _ in range(L)]
    for a, (kc, vc) in zip(layers, caches):
        a.k_cache, a.v_cache = kc.to(dev), vc.to(dev)
    # prefill of all prompt tokens (paged: K/V read back from the cache)
    pos = torch.cat([torch.arange(n) for n in lens])
    seq_of = torch.cat([torch.full((n,), i) for i, n in enumerate(lens)])
    slots = (bt.long()[seq_of, pos // B] * B + pos % B).to(torch.int32)
    cq = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    N = int(cq[-1])
    q = _randn((N, Hq, D), g)
    k = _randn((N, Hk, D), g)
    v = _randn((N, Hk, D), g)
    nkv.set_context(False, cq.to(dev), cq.to(dev), max(lens), max(lens), slots.to(dev), None,
                    bt.to(dev))
    for a, (kc, vc) in zip(layers, caches):
        o = a(q.to(dev), k.to(dev), v.to(dev), 0)
        store_kvcache_ref(k, v, kc, vc, slots)
        ref = varlen_prefill_ref(q.float(), kc, vc, cq, cq, D ** -0.5, block_tables=bt)
        assert (o.float().cpu() - ref).abs().max().item() <= TOL
    nkv.reset_context()
    # decode step: one new token per sequence, compression of sequences 0 and 1
    ctx = torch.tensor([n + 1 for n in lens], dtype=torch.int32)
    dpos = ctx.long() - 1
    dslots = (bt.long()[torch.arange(3), dpos // B] * B + dpos % B).to(torch.int32)
    qd, kd, vd = _randn((3, Hq, D), g), _randn((3, Hk, D), g), _randn((3, Hk, D), g)
    nkv.set_context(True, slot_mapping=dslots.to(dev), context_lens=ctx.to(dev),
                    block_tables=bt.to(dev))
    c = nkv.get_context()
    c.is_compress_step = True
    c.compress_selected_batch_indices = [0, 1]
    c.compress_base_context_lens = ctx.to(dev)
    outs = [a(qd.to(dev), kd.to(dev), vd.to(dev), i) for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    ctx_after = c.context_lens.cpu()
    evs = c.compression_events
    nkv.reset_context()
    sel = torch.tensor([0, 1])
    for i, (kc, vc) in enumerate(caches):
        store_kvcache_ref(kd, vd, kc, vc, dslots)
        # the kept window positions the GPU chose, read back from its compacted K: window
        # rows are distinct random vectors, so each kept row names its source position
        wslots, *_ = get_tail_window_and_tail_slots_ref(bt, ctx, sel, B, 4)
        kf_old = kc.view(-1, Hk * D)
        kf_new = layers[i].k_cache.cpu().view(-1, Hk * D)
        keep = torch.empty(2, 1, 513, dtype=torch.long)
        for r in range(2):
            old = {kf_old[int(sl)].view(torch.int16).numpy().tobytes(): p
                   for p, sl in enumerate(wslots[r])}
            keep[r, 0] = torch.tensor([old[kf_new[int(sl)].view(torch.int16).numpy().tobytes()]
                                       for sl in wslots[r, :513]])
        # ... is the oracle's selection on its own fp32 importance (all heads summed)
        k_sub, _ = gather_kv_by_slots_ref(kc, vc, wslots)
        imp = snapkv_importance_ref(qd.index_select(0, sel).unsqueeze(2), k_sub, 1, "fp32", "all")
        assert torch.equal(keep[:, 0, 1:-1], select_topk_ref(imp, 511)[:, 0])
        # ... and the compaction, lengths and events equal the oracle's for that selection
        ctx_ref = ctx.clone()
        ok, _, ev_ref = compress_compact_ref(None, kc, vc, bt, ctx, ctx_ref, [0, 1], B, 4, 2, 1,
                                             i, L, keep_idx=keep)
        assert ok
        assert torch.equal(layers[i].k_cache.cpu(), kc)
        assert torch.equal(layers[i].v_cache.cpu(), vc)
        assert torch.equal(ctx_after, ctx_ref)
        ref = paged_decode_ref(qd.float(), kc, vc, ctx_ref, bt, D ** -0.5)
        assert (outs[i][:, 0].float().cpu() - ref).abs().max().item() <= TOL
    assert evs == ev_ref
