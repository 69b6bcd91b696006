"""head_dim 64 and 256 on the GPU vs the fp32 oracle (128, the Qwen3 head size, is what every
other GPU test runs). Decode: bf16 and fp8 caches, every KV-heads-per-wave instance the plan
picks (the batch and table width below decide it), edge context lengths. Prefill: paged
one-shot and chunked, contiguous K/V with V a view of a fused qkv row, an fp8 pool, edge
lengths. Max abs error <= 2e-2 on bf16 outputs, as for head_dim 128. Compression (the general
path: score, importance, top-k and compaction kernels): importance within rtol 1e-4 of the
oracle's fp32 SnapKV, kept sets exact given those scores, compaction bit-exact, on bf16 and
fp8 pools and through the SnapKV plug-in call. Fused q/k RMSNorm + RoPE + K/V store: to
the bar of the head_dim 128 tests (bit-exact without the norm; with it at most 0.1% of
elements one or two bf16 ulps of the row maximum away)."""
import importlib

import pytest
import torch

from oracle import fp8_ref
from oracle.attention_ref import paged_decode_ref, store_kvcache_ref, varlen_prefill_ref
from oracle.rope_ref import qk_norm_rope_store_ref, rotary_cos_sin_cache_ref
from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)

pytestmark = pytest.mark.gpu
TOL = 2e-2
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")


def _err(out, ref):
    return (out.float().cpu() - ref).abs().max().item()


# (Hq, Hk, batch, ctx_lo, ctx_hi): the large batches give the several-heads-per-wave plans
# (enough chunks per resident wave), the small ones one head per wave
DECODE_CASES = [
    (32, 8, 32, 4096, 8192),   # group 4: four heads per wave (D 64), two for fp8 at D 256
    (64, 8, 24, 4096, 8192),   # group 8: two heads per wave
    (40, 8, 24, 2048, 8192),   # group 5 (Qwen3-14B): two heads per wave
    (16, 2, 3, 100, 3000),     # one head per wave
    (12, 4, 5, 1, 700),        # group 3, short contexts
]


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("Hq,Hk,bs,lo,hi", DECODE_CASES)
def test_decode_head_dim(nkv, dev, D, Hq, Hk, bs, lo, hi):
    nb = bs * (hi // 256 + 1) + 4
    wl = wl_mod.decode_workload(bs, Hq, Hk, lo, hi, nb, seed=D + Hq, head_dim=D)
    kc, vc, ctx, bt = wl["k_cache"], wl["v_cache"], wl["context_lens"], wl["block_tables"][0]
    out = nkv.paged_decode(wl["q"].to(dev), kc.to(dev), vc.to(dev), ctx.to(dev), bt.to(dev),
                           wl["scale"])
    torch.cuda.synchronize()
    assert out.shape == (bs, Hq, D)
    ref = paged_decode_ref(wl["q"].float(), kc, vc, ctx, bt, wl["scale"])
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("Hq,Hk,bs,lo,hi", DECODE_CASES[:2] + DECODE_CASES[3:4])
def test_decode_fp8_head_dim(nkv, dev, D, Hq, Hk, bs, lo, hi):
    nb = bs * (hi // 256 + 1) + 4
    wl = wl_mod.decode_workload(bs, Hq, Hk, lo, hi, nb, seed=D + Hq + 1, head_dim=D)
    k_scale, v_scale = 0.5, 0.25
    kq = fp8_ref.fp8_quantize_ref(wl["k_cache"], k_scale)
    vq = fp8_ref.fp8_quantize_ref(wl["v_cache"], v_scale)
    kf = kq.view(torch.float8_e4m3fn).float() * k_scale
    vf = vq.view(torch.float8_e4m3fn).float() * v_scale
    ctx, bt = wl["context_lens"], wl["block_tables"][0]
    out = nkv.paged_decode(wl["q"].to(dev), kq.to(dev).view(torch.float8_e4m3fn),
                           vq.to(dev).view(torch.float8_e4m3fn), ctx.to(dev), bt.to(dev),
                           wl["scale"], k_scale=k_scale, v_scale=v_scale)
    torch.cuda.synchronize()
    ref = paged_decode_ref(wl["q"].float(), kf, vf, ctx, bt, wl["scale"])
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("D", [64, 256])
def test_decode_head_dim_edge_lengths(nkv, dev, D):
    g = torch.Generator().manual_seed(D)
    nb, B, Hk = 12, 256, 4
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
    q = torch.randn(8, 16, D, generator=g).to(torch.bfloat16)
    out = nkv.paged_decode(q.to(dev), kc.to(dev), vc.to(dev), ctx.to(dev), bt.to(dev),
                           D ** -0.5)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.float(), kc, vc, ctx, bt, D ** -0.5)
    assert _err(out, ref) <= TOL
    assert torch.all(out[0] == 0)  # empty context -> zeros
    # ctx = 1 -> exactly the first value row (softmax weight 1)
    assert torch.equal(out[1, :4].cpu(), vc[int(bt[1, 0]), 0, 0].expand(4, D))


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("Hq,Hk", [(32, 8), (64, 4), (40, 8), (16, 16), (48, 4)])
def test_prefill_paged_head_dim(nkv, dev, D, Hq, Hk):
    wl = wl_mod.prefill_workload(3, Hq, Hk, 1, 500, seed=D + Hq, head_dim=D)
    kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, wl["slot_mapping"])
    out = nkv.varlen_prefill(wl["q"].to(dev), kc.to(dev), vc.to(dev), wl["cu_seqlens_q"].to(dev),
                             wl["cu_seqlens_k"].to(dev), wl["max_seqlen_q"], wl["scale"],
                             block_tables=wl["block_tables"].to(dev))
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(wl["q"].float(), kc, vc, wl["cu_seqlens_q"], wl["cu_seqlens_k"],
                             wl["scale"], block_tables=wl["block_tables"])
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("D", [64, 256])
def test_prefill_chunked_head_dim(nkv, dev, D):
    """Chunks of 200 queries after random prefixes (bottom-right causal alignment), then the
    same over an fp8 copy of the pool."""
    wl = wl_mod.prefill_workload(3, 32, 8, 0, 0, seed=D, prefix_lo=0, prefix_hi=900, chunk=200,
                                 head_dim=D)
    kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, wl["slot_mapping"])
    args = (wl["cu_seqlens_q"].to(dev), wl["cu_seqlens_k"].to(dev), wl["max_seqlen_q"],
            wl["scale"])
    bt = wl["block_tables"]
    out = nkv.varlen_prefill(wl["q"].to(dev), kc.to(dev), vc.to(dev), *args,
                             block_tables=bt.to(dev))
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(wl["q"].float(), kc, vc, wl["cu_seqlens_q"], wl["cu_seqlens_k"],
                             wl["scale"], block_tables=bt)
    assert _err(out, ref) <= TOL
    kq, vq = fp8_ref.fp8_quantize_ref(kc, 0.5), fp8_ref.fp8_quantize_ref(vc, 2.0)
    out8 = nkv.varlen_prefill(wl["q"].to(dev), kq.to(dev).view(torch.float8_e4m3fn),
                              vq.to(dev).view(torch.float8_e4m3fn), *args,
                              block_tables=bt.to(dev), max_seqlen_k=wl["max_seqlen_k"],
                              k_scale=0.5, v_scale=2.0)
    torch.cuda.synchronize()
    kf = kq.view(torch.float8_e4m3fn).float() * 0.5
    vf = vq.view(torch.float8_e4m3fn).float() * 2.0
    ref8 = varlen_prefill_ref(wl["q"].float(), kf, vf, wl["cu_seqlens_q"], wl["cu_seqlens_k"],
                              wl["scale"], block_tables=bt)
    assert _err(out8, ref8) <= TOL


@pytest.mark.parametrize("D", [64, 256])
def test_prefill_contiguous_head_dim(nkv, dev, D):
    """No block table: K roped into its own rows, V a view of a fused qkv row (its own
    stride), q a view of the same rows."""
    g = torch.Generator().manual_seed(D + 5)
    Hq, Hk = 16, 4
    Lq = [1, 37, 300, 65]
    cu = torch.tensor([0] + torch.tensor(Lq).cumsum(0).tolist(), dtype=torch.int32)
    N = int(cu[-1])
    qkv = torch.randn(N, (Hq + 2 * Hk) * D, generator=g).to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(N, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hk) * D].contiguous().view(N, Hk, D)
    v = qkv[:, (Hq + Hk) * D:].view(N, Hk, D)
    qg = qkv.to(dev)
    qd = qg[:, :Hq * D].view(N, Hq, D)
    vd = qg[:, (Hq + Hk) * D:].view(N, Hk, D)
    out = nkv.varlen_prefill(qd, k.to(dev), vd, cu.to(dev), cu.to(dev), max(Lq), D ** -0.5)
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(q.float(), k, v.contiguous(), cu, cu, D ** -0.5)
    assert _err(out, ref) <= TOL


@pytest.mark.parametrize("D", [64, 256])
def test_prefill_edge_lengths_head_dim(nkv, dev, D):
    """Empty, single-token and tile-boundary sequences; Lk < Lq rows are zero."""
    g = torch.Generator().manual_seed(D + 14)
    Hq, Hk = 32, 8
    Lq = [0, 1, 31, 32, 33, 127, 128, 129, 5, 40]
    Lk = [0, 1, 31, 32, 33, 127, 128, 129, 300, 17]  # last: 23 queries see nothing
    cu_q = torch.tensor([0] + torch.tensor(Lq).cumsum(0).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + torch.tensor(Lk).cumsum(0).tolist(), dtype=torch.int32)
    q = torch.randn(int(cu_q[-1]), Hq, D, generator=g).to(torch.bfloat16)
    k = torch.randn(int(cu_k[-1]), Hk, D, generator=g).to(torch.bfloat16)
    v = torch.randn(int(cu_k[-1]), Hk, D, generator=g).to(torch.bfloat16)
    out = nkv.varlen_prefill(q.to(dev), k.to(dev), v.to(dev), cu_q.to(dev), cu_k.to(dev),
                             max(Lq), D ** -0.5)
    torch.cuda.synchronize()
    ref = varlen_prefill_ref(q.float(), k, v, cu_q, cu_k, D ** -0.5)
    assert _err(out, ref) <= TOL
    o = out.cpu()
    last = int(cu_q[-2])
    assert torch.all(o[last:last + 23] == 0)
    assert torch.equal(o[0], v[0].repeat_interleave(Hq // Hk, dim=0))


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("agg", ["all", "group"])
@pytest.mark.parametrize("D", [64, 256])
def test_compress_step_head_dim(nkv, dev, D, agg, fp8):
    """A compression step (window of 4 blocks, keep 2*256+1) with a -1 padding entry in
    seq_idx, on a bf16 or an fp8 pool."""
    W, KEEP, ks, vs = 4, 2 * 256 + 1, 0.5, 2.0
    wl = wl_mod.compress_workload(24, 32, 8, 1500, 4096, 5, 4 + D, selected_only=True,
                                  head_dim=D)
    if fp8:
        kq = fp8_ref.fp8_quantize_ref(wl["k_cache"], ks)
        vq = fp8_ref.fp8_quantize_ref(wl["v_cache"], vs)
        kg = kq.to(dev).view(torch.float8_e4m3fn)
        vg = vq.to(dev).view(torch.float8_e4m3fn)
        kf = kq.view(torch.float8_e4m3fn).float() * ks
    else:
        kg, vg = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
        kf = wl["k_cache"]
    sel = wl["seq_idx"]
    seq_idx = torch.tensor(sel[:2] + [-1] + sel[2:], dtype=torch.int32, device=dev)
    base = wl["context_lens"].to(dev)
    ctx = base.clone()
    keep, imp = cu.compress_step(wl["q"].to(dev), kg, vg, wl["block_tables"].to(dev), base, ctx,
                                 seq_idx, W, KEEP, D ** -0.5, agg,
                                 **({"k_scale": ks} if fp8 else {}))
    torch.cuda.synchronize()
    real = [i for i in range(seq_idx.numel()) if i != 2]
    imp, keep = imp.cpu()[real], keep.cpu()[real]
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(wl["block_tables"], wl["context_lens"], st,
                                                   256, W)
    k_sub, _ = gather_kv_by_slots_ref(kf, kf, slots)
    ref_imp = snapkv_importance_ref(wl["q"].index_select(0, st).unsqueeze(2), k_sub, 1, "fp32",
                                    agg)
    assert torch.allclose(imp, ref_imp, rtol=1e-4, atol=1e-7)
    assert torch.equal(keep[..., 1:-1].long(), select_topk_ref(imp, KEEP - 2))
    if fp8:
        kc, vc = kq.clone(), vq.clone()
    else:
        kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    ctx_ref = wl["context_lens"].clone()
    ok, _, _ = compress_compact_ref(None, kc, vc, wl["block_tables"], wl["context_lens"], ctx_ref,
                                    sel, 256, W, 2, 1, 0, 1, keep_idx=keep.long())
    assert ok
    got_k = kg.view(torch.uint8).cpu() if fp8 else kg.cpu()
    got_v = vg.view(torch.uint8).cpu() if fp8 else vg.cpu()
    assert torch.equal(got_k, kc) and torch.equal(got_v, vc)
    assert torch.equal(ctx.cpu(), ctx_ref)


@pytest.mark.parametrize("window", [1, 5])
@pytest.mark.parametrize("D", [64, 256])
def test_snapkv_head_dim(nkv, dev, D, window):
    """SnapKV(Q, K, V, num_keep, window) on contiguous [m, H, L, D] tensors."""
    g = torch.Generator().manual_seed(D + window)
    L, agg = 1024, "group"
    Q = torch.randn(2, 16, window, D, generator=g).to(torch.bfloat16)
    K = torch.randn(2, 4, L, D, generator=g).to(torch.bfloat16)
    num_keep = L // 2 - 1
    out, imp = nkv.SnapKV(Q.to(dev), K.to(dev), None, num_keep=num_keep, window=window, agg=agg,
                          return_importance=True)
    torch.cuda.synchronize()
    out = out.cpu().view(2, 4, num_keep + 1 + window)
    ref_imp = snapkv_importance_ref(Q, K, window, "fp32", agg)
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    assert torch.equal(out[..., 1:num_keep + 1], select_topk_ref(imp.cpu(), num_keep))
    assert torch.equal(out[..., num_keep + 1:], torch.arange(L - window, L).expand(2, 4, window))


def _rope_close(out, ref):
    out, ref = out.float().cpu(), ref.float()
    rowmax = ref.abs().amax(dim=-1, keepdim=True)
    diff = (out - ref).abs()
    assert torch.all(diff <= rowmax * 2.0 ** -6), f"max diff {diff.max().item()}"
    assert (diff > 0).float().mean().item() <= 1e-3


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("Hq,Hk", [(32, 8), (8, 1)])
def test_norm_rope_store_head_dim(nkv, dev, D, Hq, Hk):
    g = torch.Generator().manual_seed(D + Hq)
    N, nb, B, max_pos = 300, 8, 256, 40960
    qkv = (torch.randn(N, (Hq + 2 * Hk) * D, generator=g) * 3.0).to(torch.bfloat16)
    qw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    pos = torch.randint(0, max_pos, (N,), generator=g)
    cache = rotary_cos_sin_cache_ref(D, max_pos, 1e6)
    kc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, B, Hk, D, generator=g).to(torch.bfloat16)
    slots = torch.randperm(nb * B, generator=g)[:N].to(torch.int32)
    slots[5] = -1
    kg, vg = kc.to(dev), vc.to(dev)
    qkvg = qkv.to(dev)
    q = qkvg[:, :Hq * D].view(N, Hq, D)
    k = qkvg[:, Hq * D:(Hq + Hk) * D].view(N, Hk, D)
    v = qkvg[:, (Hq + Hk) * D:].view(N, Hk, D)
    qo, ko, _ = nkv.qk_norm_rope_store(pos.to(dev), q, k, v, cache.to(dev), qw.to(dev),
                                       kw.to(dev), 1e-6, k_cache=kg, v_cache=vg,
                                       slot_mapping=slots.to(dev))
    torch.cuda.synchronize()
    qr, kr, _ = qk_norm_rope_store_ref(qkv, pos, qw, kw, 1e-6, cache, Hq, Hk, head_dim=D,
                                       k_cache=kc, v_cache=vc, slot_mapping=slots)
    _rope_close(qo, qr)
    _rope_close(ko, kr)
    _rope_close(kg.cpu().view(-1, Hk, D), kc.view(-1, Hk, D))
    assert torch.equal(vg.cpu(), vc)
    # without the norm: bit-exact
    qo2, ko2, _ = nkv.qk_norm_rope_store(pos.to(dev), q, k, None, cache.to(dev))
    torch.cuda.synchronize()
    qr2, kr2, _ = qk_norm_rope_store_ref(qkv, pos, None, None, 0.0, cache, Hq, Hk, head_dim=D)
    assert torch.equal(qo2.cpu(), qr2) and torch.equal(ko2.cpu(), kr2)


@pytest.mark.parametrize("D", [64, 256])
def test_attention_module_head_dim(nkv, dev, D):
    """Attention.forward with head_dim 64 / 256: the decode branch (store, then attend) and
    the prefill branch (store, then varlen attention over the paged cache)."""
    from types import SimpleNamespace
    cfg = SimpleNamespace(kv_compress_enabled=False)
    wl = wl_mod.decode_workload(4, 16, 8, 300, 1000, 16, seed=D, value_scale=D ** -0.5,
                                head_dim=D)
    attn = nkv.Attention(16, D, D ** -0.5, 8, cfg, 1)
    attn.k_cache, attn.v_cache = wl["k_cache"].to(dev), wl["v_cache"].to(dev)
    bt, slots = wl["block_tables"][0], wl["slot_mappings"][0]
    nkv.set_context(True, slot_mapping=slots.to(dev), context_lens=wl["context_lens"].to(dev),
                    block_tables=bt.to(dev))
    o = attn(wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev), 0)
    nkv.reset_context()
    kc, vc = wl["k_cache"].clone(), wl["v_cache"].clone()
    store_kvcache_ref(wl["key"], wl["value"], kc, vc, slots)
    ref = paged_decode_ref(wl["q"].float(), kc, vc, wl["context_lens"], bt, wl["scale"])
    assert o.shape == (4, 1, 16, D)
    assert _err(o[:, 0], ref) <= TOL

    pw = wl_mod.prefill_workload(3, 16, 8, 0, 0, seed=D + 1, prefix_lo=0, prefix_hi=600,
                                 chunk=100, head_dim=D)
    attn.k_cache, attn.v_cache = pw["k_cache"].to(dev), pw["v_cache"].to(dev)
    nkv.set_context(False, cu_seqlens_q=pw["cu_seqlens_q"].to(dev),
                    cu_seqlens_k=pw["cu_seqlens_k"].to(dev), max_seqlen_q=pw["max_seqlen_q"],
                    max_seqlen_k=pw["max_seqlen_k"], slot_mapping=pw["slot_mapping"].to(dev),
                    block_tables=pw["block_tables"].to(dev))
    o = attn(pw["q"].to(dev), pw["key"].to(dev), pw["value"].to(dev), 0)
    nkv.reset_context()
    kc, vc = pw["k_cache"].clone(), pw["v_cache"].clone()
    store_kvcache_ref(pw["key"], pw["value"], kc, vc, pw["slot_mapping"])
    ref = varlen_prefill_ref(pw["q"].float(), kc, vc, pw["cu_seqlens_q"], pw["cu_seqlens_k"],
                             pw["scale"], block_tables=pw["block_tables"])
    assert _err(o.view(ref.shape), ref) <= TOL
