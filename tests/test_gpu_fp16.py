"""fp16 models: every kernel family with fp16 q/K/V/outputs against the oracle.

The reference allocates its K/V pool in the checkpoint's dtype
(torch.set_default_dtype(hf_config.torch_dtype), nanokvllm/engine/model_runner.py:27,
142-145) and hands fp16 tensors to flash-attn (nanokvllm/layers/attention.py:96-107), e.g.
for the fp16 AWQ checkpoints of docs/AWQ_bug.md:335-348. The oracle runs in fp32 on the same
fp16 inputs. Bars as in the bf16 suite: attention outputs within 2e-2 of the oracle (the
outputs are fp16); the store bit-exact; importance within rtol 1e-4, kept sets exact given
the scores, compaction, lengths and events bit-exact; norm + RoPE bit-exact without the norm,
and with it at most 0.1% of elements off, each by at most 2 fp16 ulps of the row's maximum.
"""
import importlib
import random
from types import SimpleNamespace

import pytest
import torch

from oracle.attention_ref import (paged_decode_ref, store_kvcache_ref, varlen_prefill_ref)
from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)
from oracle.rope_ref import qk_norm_rope_store_ref, rotary_cos_sin_cache_ref

pytestmark = pytest.mark.gpu
TOL = 2e-2
F16 = torch.float16
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
kv_mod = importlib.import_module("nanokv-llm_amd.layers.kv_cache")


def _h(x):
    return x.to(F16)


def test_store_fp16_bit_exact(nkv, dev):
    g = torch.Generator().manual_seed(1)
    N, Hk, D, nb, B = 300, 8, 128, 6, 256
    key, value = _h(torch.randn(N, Hk, D, generator=g)), _h(torch.randn(N, Hk, D, generator=g))
    kc, vc = _h(torch.randn(nb, B, Hk, D, generator=g)), _h(torch.randn(nb, B, Hk, D, generator=g))
    slots = torch.randperm(nb * B, generator=g)[:N].to(torch.int32)
    slots[::7] = -1
    kg, vg = kc.to(dev), vc.to(dev)
    nkv.store_kvcache(key.to(dev), value.to(dev), kg, vg, slots.to(dev))
    torch.cuda.synchronize()
    store_kvcache_ref(key, value, kc, vc, slots)
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)


@pytest.mark.parametrize("Hq,Hk,D", [(32, 8, 128), (16, 8, 64), (8, 2, 256), (40, 8, 128),
                                     (64, 2, 128)])
def test_decode_fp16(nkv, dev, Hq, Hk, D):
    """Table widths below and above the two-heads-per-wave threshold; g = 32 takes the
    column-group split."""
    for width_blocks, bs, hi in ((4, 9, 1000), (32, 24, 8000)):
        wl = wl_mod.decode_workload(bs, Hq, Hk, 1, hi, bs * width_blocks + 8,
                                    seed=Hq * 10 + Hk + D + width_blocks, head_dim=D)
        q, kc, vc = _h(wl["q"]), _h(wl["k_cache"]), _h(wl["v_cache"])
        bt, ctx = wl["block_tables"][0], wl["context_lens"]
        print(f"fp16 decode Hq={Hq} Hk={Hk} D={D} bs={bs}", flush=True)
        out = nkv.paged_decode(q.to(dev), kc.to(dev), vc.to(dev), ctx.to(dev), bt.to(dev),
                               D ** -0.5)
        torch.cuda.synchronize()
        assert out.dtype == F16
        ref = paged_decode_ref(q.float(), kc, vc, ctx, bt, D ** -0.5)
        assert (out.float().cpu() - ref).abs().max().item() <= TOL


def test_decode_fp16_qwen3_8b_geometry(nkv, dev):
    """The benchmarked decode shape (batch 64, Hq 32, Hk 8, ctx U[2048, 8192]) in fp16: the
    new token stored, then 16 of the 64 sequences against the oracle."""
    wl = wl_mod.decode_qwen3_8b(seed=2, device=dev)
    kc, vc = _h(wl["k_cache"]), _h(wl["v_cache"])
    bt, slots = wl["block_tables"][0].to(dev), wl["slot_mappings"][0].to(dev)
    q, ctx = _h(wl["q"]).to(dev), wl["context_lens"].to(dev)
    nkv.store_kvcache(_h(wl["key"]).to(dev), _h(wl["value"]).to(dev), kc, vc, slots)
    out = nkv.paged_decode(q, kc, vc, ctx, bt, wl["scale"])
    torch.cuda.synchronize()
    rows = torch.arange(0, 64, 4)
    ids = sorted({int(x) for x in bt.cpu()[rows].flatten().tolist() if x >= 0})
    remap = {b: j for j, b in enumerate(ids)}
    idx = torch.tensor(ids, device=dev)
    kh, vh = kc.index_select(0, idx).cpu(), vc.index_select(0, idx).cpu()
    bt2 = torch.tensor([[remap.get(int(x), -1) for x in r] for r in bt.cpu()[rows].tolist()],
                       dtype=torch.int32)
    ref = paged_decode_ref(q.cpu()[rows].float(), kh, vh, ctx.cpu()[rows], bt2, wl["scale"])
    assert (out.cpu()[rows].float() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("Hq,Hk,D", [(32, 8, 128), (16, 8, 64), (16, 4, 256)])
def test_prefill_fp16_paged_chunked(nkv, dev, Hq, Hk, D):
    wl = wl_mod.prefill_workload(4, Hq, Hk, 0, 0, seed=40 + Hq + D, prefix_lo=0, prefix_hi=900,
                                 chunk=200, head_dim=D)
    q, key, value = _h(wl["q"]), _h(wl["key"]), _h(wl["value"])
    kc, vc = _h(wl["k_cache"]), _h(wl["v_cache"])
    store_kvcache_ref(key, value, kc, vc, wl["slot_mapping"])
    out = nkv.varlen_prefill(q.to(dev), kc.to(dev), vc.to(dev), wl["cu_seqlens_q"].to(dev),
                             wl["cu_seqlens_k"].to(dev), wl["max_seqlen_q"], D ** -0.5,
                             block_tables=wl["block_tables"].to(dev))
    torch.cuda.synchronize()
    assert out.dtype == F16
    ref = varlen_prefill_ref(q.float(), kc, vc, wl["cu_seqlens_q"], wl["cu_seqlens_k"],
                             D ** -0.5, block_tables=wl["block_tables"])
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


def test_prefill_fp16_contiguous(nkv, dev):
    wl = wl_mod.prefill_workload(3, 32, 8, 1, 700, seed=43)
    q, k, v = _h(wl["q"]), _h(wl["key"]), _h(wl["value"])
    cq = wl["cu_seqlens_q"]
    out = nkv.varlen_prefill(q.to(dev), k.to(dev), v.to(dev), cq.to(dev), cq.to(dev),
                             wl["max_seqlen_q"], 128 ** -0.5)
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(q.float(), k, v, cq, cq, 128 ** -0.5)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("agg", ["group", "all"])
@pytest.mark.parametrize("Hq,Hk", [(32, 8), (64, 2)])
def test_compress_step_fp16(nkv, dev, agg, Hq, Hk):
    """The compression step on an fp16 pool (fused kernels at g = 4, the score / top-k /
    compaction kernels at g = 32) with compress_finalize's table and slot rewrite."""
    wl = wl_mod.compress_workload(60, Hq, Hk, 1500, 4096, 6, seed=Hq + Hk + 7,
                                  selected_only=True)
    bt, base, sel = wl["block_tables"], wl["context_lens"], wl["seq_idx"]
    q, kc, vc = _h(wl["q"]), _h(wl["k_cache"]), _h(wl["v_cache"])
    print(f"fp16 compression Hq={Hq} Hk={Hk} agg={agg}", flush=True)
    kg, vg, btg = kc.to(dev), vc.to(dev), bt.to(dev)
    ctx = base.clone().to(dev)
    seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
    keep, imp = cu.compress_step(q.to(dev), kg, vg, btg, base.to(dev), ctx, seq_idx, 4, 513,
                                 128 ** -0.5, agg)
    events = torch.empty(len(sel), 4 + bt.size(1), dtype=torch.int32, device=dev)
    cu.compress_finalize(btg, base.to(dev), seq_idx, 513, 256, 4, events, rewrite_tables=True)
    torch.cuda.synchronize()
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt, base, st, 256, 4)
    k_sub, _ = gather_kv_by_slots_ref(kc, vc, slots)
    ref_imp = snapkv_importance_ref(q.index_select(0, st).unsqueeze(2), k_sub, 1, "fp32", agg)
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    keep = keep.cpu().long()
    assert torch.equal(keep[..., 1:-1], select_topk_ref(imp.cpu(), 511))
    kr, vr, ctx_ref = kc.clone(), vc.clone(), base.clone()
    ok, _, ev_ref = compress_compact_ref(None, kr, vr, bt, base, ctx_ref, sel, 256, 4, 2, 1, 0,
                                         1, keep_idx=keep)
    assert ok
    assert torch.equal(kg.cpu(), kr) and torch.equal(vg.cpu(), vr)
    assert torch.equal(ctx.cpu(), ctx_ref)
    assert cu.events_to_dicts(events, 0) == ev_ref


@pytest.mark.parametrize("window,L", [(1, 1024), (5, 1000), (1, 333)])
def test_snapkv_fp16(nkv, dev, window, L):
    g = torch.Generator().manual_seed(window + L)
    Q = _h(torch.randn(3, 32, window, 128, generator=g))
    K = _h(torch.randn(3, 8, L, 128, generator=g))
    num_keep = L // 2 - 1
    out, imp = nkv.SnapKV(Q.to(dev), K.to(dev), None, num_keep=num_keep, window=window,
                          agg="all", return_importance=True)
    torch.cuda.synchronize()
    ref_imp = snapkv_importance_ref(Q, K, window, "fp32", "all")
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    out = out.cpu().view(3, 1, num_keep + 1 + window)
    assert torch.equal(out[..., 1:num_keep + 1], select_topk_ref(imp.cpu(), num_keep))


def _rope_case(N, Hq, Hk, seed, D=128, nb=8, B=256, max_pos=40960, scale=3.0):
    g = torch.Generator().manual_seed(seed)
    qkv = _h(torch.randn(N, (Hq + 2 * Hk) * D, generator=g) * scale)
    qw = _h(1 + 0.3 * torch.randn(D, generator=g))
    kw = _h(1 + 0.3 * torch.randn(D, generator=g))
    pos = torch.randint(0, max_pos, (N,), generator=g)
    cache = rotary_cos_sin_cache_ref(D, max_pos, 1e6)
    kc, vc = _h(torch.randn(nb, B, Hk, D, generator=g)), _h(torch.randn(nb, B, Hk, D, generator=g))
    slots = torch.randperm(nb * B, generator=g)[:N].to(torch.int32)
    slots[0] = -1
    return qkv, qw, kw, pos, cache, kc, vc, slots


def _close16(out, ref):
    out, ref = out.float().cpu(), ref.float()
    rowmax = ref.abs().amax(dim=-1, keepdim=True)
    diff = (out - ref).abs()
    assert torch.all(diff <= rowmax * 2.0 ** -9), f"max diff {diff.max().item()}"
    assert (diff > 0).float().mean().item() <= 1e-3


def test_qk_norm_rope_store_fp16(nkv, dev):
    N, Hq, Hk, D = 300, 32, 8, 128
    qkv, qw, kw, pos, cache, kc, vc, slots = _rope_case(N, Hq, Hk, seed=5)
    kg, vg = kc.to(dev), vc.to(dev)
    qkvg = qkv.to(dev)
    q, k, v = (qkvg[:, :Hq * D].view(N, Hq, D), qkvg[:, Hq * D:(Hq + Hk) * D].view(N, Hk, D),
               qkvg[:, (Hq + Hk) * D:].view(N, Hk, D))
    qo, ko, _ = nkv.qk_norm_rope_store(pos.to(dev), q, k, v, cache.to(dev), qw.to(dev),
                                       kw.to(dev), 1e-6, k_cache=kg, v_cache=vg,
                                       slot_mapping=slots.to(dev))
    torch.cuda.synchronize()
    assert qo.dtype == F16 and ko.dtype == F16
    qr, kr, _ = qk_norm_rope_store_ref(qkv, pos, qw, kw, 1e-6, cache, Hq, Hk, k_cache=kc,
                                       v_cache=vc, slot_mapping=slots)
    _close16(qo, qr)
    _close16(ko, kr)
    assert torch.equal(vg.cpu(), vc)
    # without the norm: bit-exact
    qo2, ko2, _ = nkv.qk_norm_rope_store(pos.to(dev), q, k, None, cache.to(dev), need_k=True)
    torch.cuda.synchronize()
    qr2, kr2, _ = qk_norm_rope_store_ref(qkv, pos, None, None, 1e-6, cache, Hq, Hk)
    assert torch.equal(qo2.cpu(), qr2) and torch.equal(ko2.cpu(), kr2)


def test_attention_fp16_pool_flow(nkv, dev):
    """Two fp16 Attention layers over an fp16 KVCachePool: a prefill step, then a decode step
    with a compression step (agg "all"), through Attention.forward, against the oracle."""
    g = torch.Generator().manual_seed(16)
    Hq, Hk, D, B, L = 32, 8, 128, 256, 2
    cfg = SimpleNamespace(kv_compress_enabled=True, kv_compress_window_blocks=4,
                          kv_compress_keep_blocks=2, kv_compress_keep_extra_tokens=1)
    layers = [nkv.Attention(Hq, D, D ** -0.5, Hk, cfg, L) for _ in range(L)]
    pool = kv_mod.KVCachePool(L, Hk, D, B, dtype=F16, num_blocks=40, device=dev)
    assert pool.bind(layers) == L
    for a in layers:
        a.k_cache.copy_(_h(torch.randn(a.k_cache.shape, generator=g)))
        a.v_cache.copy_(_h(torch.randn(a.v_cache.shape, generator=g)))
    caches = [(a.k_cache.cpu(), a.v_cache.cpu()) for a in layers]
    lens = [1300, 2100]
    rng = random.Random(16)
    free = list(range(40))
    rng.shuffle(free)
    bt = torch.full((2, 12), -1, dtype=torch.int32)
    for i, n in enumerate(lens):
        nbk = (n + 1 + B - 1) // B
        bt[i, :nbk] = torch.tensor([free.pop() for _ in range(nbk)])
    pos = torch.cat([torch.arange(n) for n in lens])
    seq_of = torch.cat([torch.full((n,), i) for i, n in enumerate(lens)])
    slots = (bt.long()[seq_of, pos // B] * B + pos % B).to(torch.int32)
    cq = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32)
    N = int(cq[-1])
    q, k, v = (_h(torch.randn(N, Hq, D, generator=g)), _h(torch.randn(N, Hk, D, generator=g)),
               _h(torch.randn(N, Hk, D, generator=g)))
    nkv.set_context(False, cq.to(dev), cq.to(dev), max(lens), max(lens), slots.to(dev), None,
                    bt.to(dev))
    for a, (kc, vc) in zip(layers, caches):
        o = a(q.to(dev), k.to(dev), v.to(dev), 0)
        assert o.dtype == F16
        store_kvcache_ref(k, v, kc, vc, slots)
        ref = varlen_prefill_ref(q.float(), kc, vc, cq, cq, D ** -0.5, block_tables=bt)
        assert (o.float().cpu() - ref).abs().max().item() <= TOL
    nkv.reset_context()
    ctx = torch.tensor([n + 1 for n in lens], dtype=torch.int32)
    dpos = ctx.long() - 1
    dslots = (bt.long()[torch.arange(2), dpos // B] * B + dpos % B).to(torch.int32)
    qd, kd, vd = (_h(torch.randn(2, Hq, D, generator=g)), _h(torch.randn(2, Hk, D, generator=g)),
                  _h(torch.randn(2, Hk, D, generator=g)))
    nkv.set_context(True, slot_mapping=dslots.to(dev), context_lens=ctx.to(dev),
                    block_tables=bt.to(dev))
    c = nkv.get_context()
    c.is_compress_step = True
    c.compress_selected_batch_indices = [0, 1]
    c.compress_base_context_lens = ctx.to(dev)
    outs = [a(qd.to(dev), kd.to(dev), vd.to(dev), i) for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    ctx_after = c.context_lens.cpu()
    nkv.reset_context()
    sel = torch.tensor([0, 1])
    for i, (kc, vc) in enumerate(caches):
        store_kvcache_ref(kd, vd, kc, vc, dslots)
        wslots, *_ = get_tail_window_and_tail_slots_ref(bt, ctx, sel, B, 4)
        k_sub, _ = gather_kv_by_slots_ref(kc, vc, wslots)
        imp = snapkv_importance_ref(qd.index_select(0, sel).unsqueeze(2), k_sub, 1, "fp32", "all")
        keep = torch.cat([torch.zeros(2, 1, 1, dtype=torch.long), select_topk_ref(imp, 511),
                          torch.full((2, 1, 1), 1023, dtype=torch.long)], dim=-1)
        ctx_ref = ctx.clone()
        ok, _, _ = compress_compact_ref(None, kc, vc, bt, ctx, ctx_ref, [0, 1], B, 4, 2, 1, i, L,
                                        keep_idx=keep)
        assert ok
        assert torch.equal(layers[i].k_cache.cpu(), kc)
        assert torch.equal(layers[i].v_cache.cpu(), vc)
        assert torch.equal(ctx_after, ctx_ref)
        ref = paged_decode_ref(qd.float(), kc, vc, ctx_ref, bt, D ** -0.5)
        assert (outs[i][:, 0].float().cpu() - ref).abs().max().item() <= TOL
    del pool, layers
