"""fp8 (OCP E4M3FN) K/V on the GPU vs the oracle: conversions bit-exact over every code and
every bf16 input (including clamping and NaN), store bit-exact."""
import importlib

import pytest
import torch

from oracle import fp8_ref

pytestmark = pytest.mark.gpu
kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")


def test_dequantize_every_code(nkv, dev):
    codes = torch.arange(256, dtype=torch.uint8)
    for scale in (1.0, 0.37):
        out = kvc.fp8_dequantize(codes.to(dev), scale).cpu()
        ref = fp8_ref.fp8_dequantize_ref(codes, scale)
        nan = torch.isnan(ref.float())
        assert torch.equal(torch.isnan(out.float()), nan)
        assert torch.equal(out[~nan], ref[~nan])


def test_quantize_every_bf16(nkv, dev):
    x = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    for scale in (1.0, 0.37, 3.0):
        got = kvc.fp8_quantize(x.to(dev), scale).view(torch.uint8).cpu()
        ref = fp8_ref.fp8_quantize_ref(x, scale)
        nan = torch.isnan(x.float())
        assert torch.equal(got[~nan], ref[~nan]), f"scale {scale}"
        assert set(got[nan].tolist()) <= {0x7F, 0xFF}


def test_store_fp8(nkv, dev):
    g = torch.Generator().manual_seed(3)
    N, Hq, Hk, D, nb, B = 37, 32, 8, 128, 6, 256
    qkv = torch.randn(N, (Hq + 2 * Hk) * D, generator=g).to(torch.bfloat16)
    key = qkv[:, Hq * D:(Hq + Hk) * D].view(N, Hk, D)
    value = qkv[:, (Hq + Hk) * D:].view(N, Hk, D)
    kc = torch.randint(0, 255, (nb, B, Hk, D), generator=g, dtype=torch.uint8)
    vc = torch.randint(0, 255, (nb, B, Hk, D), generator=g, dtype=torch.uint8)
    slots = torch.randperm(nb * B, generator=g)[:N].to(torch.int32)
    slots[[0, 9]] = -1
    kg, vg = kc.to(dev).view(torch.float8_e4m3fn), vc.to(dev).view(torch.float8_e4m3fn)
    qg = qkv.to(dev)
    nkv.store_kvcache(qg[:, Hq * D:(Hq + Hk) * D].view(N, Hk, D),
                      qg[:, (Hq + Hk) * D:].view(N, Hk, D), kg, vg, slots.to(dev), 0.5, 2.0)
    torch.cuda.synchronize()
    fp8_ref.store_kvcache_fp8_ref(key, value, kc, vc, slots, 0.5, 2.0)
    assert torch.equal(kg.view(torch.uint8).cpu(), kc) and torch.equal(vg.view(torch.uint8).cpu(), vc)


wl_mod = importlib.import_module("nanokv-llm_amd.workloads")


def _fp8_state(Hq, Hk, bs=6, seed=5, lo=1, hi=8192):
    wl = wl_mod.decode_workload(bs, Hq, Hk, lo, hi, bs * 32 + 4, seed=seed)
    return wl


@pytest.mark.parametrize("Hq,Hk", [(32, 8), (8, 8), (16, 8), (64, 8), (128, 8), (16, 2)])
def test_decode_fp8_equals_bf16_over_dequantized(nkv, dev, Hq, Hk):
    """Scales 1: the fp8 kernel widens codes to the same bf16 values the bf16 kernel reads.
    Where both group the KV heads alike, the outputs are equal bit for bit. Where fp8 takes
    four KV heads per wave (Hk % 4 == 0, group <= 4, a table this wide) and bf16 two, the
    chunk stream is split at other points and the two agree within 1e-2."""
    wl = _fp8_state(Hq, Hk)
    kq = kvc.fp8_quantize(wl["k_cache"].to(dev))
    vq = kvc.fp8_quantize(wl["v_cache"].to(dev))
    kd, vd = kvc.fp8_dequantize(kq), kvc.fp8_dequantize(vq)
    args = (wl["context_lens"].to(dev), wl["block_tables"][0].to(dev), wl["scale"])
    q = wl["q"].to(dev)
    a = nkv.paged_decode(q, kq, vq, *args)
    b = nkv.paged_decode(q, kd, vd, *args)
    if Hk % 4 == 0 and Hq // Hk <= 4:
        assert (a.float() - b.float()).abs().max().item() <= 1e-2
    else:
        assert torch.equal(a, b)


@pytest.mark.parametrize("k_scale,v_scale", [(1.0, 1.0), (0.5, 2.0), (0.037, 0.011)])
def test_decode_fp8_vs_oracle(nkv, dev, k_scale, v_scale):
    from oracle.attention_ref import paged_decode_ref
    wl = _fp8_state(32, 8, seed=6)
    kc, vc = wl["k_cache"], wl["v_cache"]
    kq = fp8_ref.fp8_quantize_ref(kc, k_scale)
    vq = fp8_ref.fp8_quantize_ref(vc, v_scale)
    kf = kq.view(torch.float8_e4m3fn).float() * k_scale  # fp32 dequantization
    vf = vq.view(torch.float8_e4m3fn).float() * v_scale
    ctx, bt = wl["context_lens"], wl["block_tables"][0]
    out = nkv.paged_decode(wl["q"].to(dev), kq.to(dev).view(torch.float8_e4m3fn),
                           vq.to(dev).view(torch.float8_e4m3fn), ctx.to(dev), bt.to(dev),
                           wl["scale"], k_scale=k_scale, v_scale=v_scale)
    ref = paged_decode_ref(wl["q"].float(), kf, vf, ctx, bt, wl["scale"])
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2


def test_attention_with_fp8_pool(nkv, dev):
    """KVCachePool(fp8) bound to two layers: store + decode through Attention.forward vs the
    oracle on the dequantized cache."""
    from types import SimpleNamespace

    from oracle.attention_ref import paged_decode_ref
    wl = _fp8_state(32, 8, bs=4, seed=7, lo=300, hi=3000)
    NB = wl["k_cache"].size(0)
    pool = kvc.KVCachePool(2, 8, 128, dtype=torch.float8_e4m3fn, num_blocks=NB, device=dev,
                           k_scale=0.25, v_scale=0.5)
    layers = [nkv.Attention(32, 128, wl["scale"], 8, SimpleNamespace(kv_compress_enabled=False),
                            2) for _ in range(2)]
    assert pool.bind(layers) == 2 and layers[1].k_scale == 0.25
    for a in layers:  # start from the workload's cache, quantized
        kvc.fp8_quantize(wl["k_cache"].to(dev), 0.25, out=a.k_cache)
        kvc.fp8_quantize(wl["v_cache"].to(dev), 0.5, out=a.v_cache)
    bt, slots, ctx = wl["block_tables"][0], wl["slot_mappings"][0], wl["context_lens"]
    nkv.set_context(True, slot_mapping=slots.to(dev), context_lens=ctx.to(dev),
                    block_tables=bt.to(dev))
    o = layers[0](wl["q"].to(dev), wl["key"].to(dev), wl["value"].to(dev), 0)
    torch.cuda.synchronize()
    nkv.reset_context()
    kq = fp8_ref.fp8_quantize_ref(wl["k_cache"], 0.25)
    vq = fp8_ref.fp8_quantize_ref(wl["v_cache"], 0.5)
    fp8_ref.store_kvcache_fp8_ref(wl["key"], wl["value"], kq, vq, slots, 0.25, 0.5)
    assert torch.equal(layers[0].k_cache.view(torch.uint8).cpu(), kq)
    ref = paged_decode_ref(wl["q"].float(), kq.view(torch.float8_e4m3fn).float() * 0.25,
                           vq.view(torch.float8_e4m3fn).float() * 0.5, ctx, bt, wl["scale"])
    assert (o.squeeze(1).float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("B", [256, 16, 48])
def test_prefill_over_fp8_pool(nkv, dev, B):
    """Chunked prefill reading a paged fp8 cache (the kernel widens the codes as it stages
    them) vs the oracle on the fp32-dequantized cache; block sizes whose 64-key steps
    cross up to 4 blocks too."""
    from oracle.attention_ref import varlen_prefill_ref
    wl = wl_mod.prefill_workload(3, 32, 8, 0, 0, seed=12, prefix_lo=0, prefix_hi=900, chunk=200,
                                 block_size=B)
    kq = fp8_ref.fp8_quantize_ref(wl["k_cache"], 0.5)
    vq = fp8_ref.fp8_quantize_ref(wl["v_cache"], 2.0)
    fp8_ref.store_kvcache_fp8_ref(wl["key"], wl["value"], kq, vq, wl["slot_mapping"], 0.5, 2.0)
    out = nkv.varlen_prefill(wl["q"].to(dev), kq.to(dev).view(torch.float8_e4m3fn),
                             vq.to(dev).view(torch.float8_e4m3fn), wl["cu_seqlens_q"].to(dev),
                             wl["cu_seqlens_k"].to(dev), wl["max_seqlen_q"], wl["scale"],
                             block_tables=wl["block_tables"].to(dev),
                             max_seqlen_k=wl["max_seqlen_k"], k_scale=0.5, v_scale=2.0)
    kf = kq.view(torch.float8_e4m3fn).float() * 0.5
    vf = vq.view(torch.float8_e4m3fn).float() * 2.0
    ref = varlen_prefill_ref(wl["q"].float(), kf, vf, wl["cu_seqlens_q"], wl["cu_seqlens_k"],
                             wl["scale"], block_tables=wl["block_tables"])
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("G", [4, 5])
def test_prefill_over_fp8_pool_mixed_batch(nkv, dev, G):
    """A mixed chunked-prefill step over an fp8 pool: decode rows (one query over a long
    context) beside prompt chunks, block size 16 and 256-token blocks' worth of context,
    within 2e-2 of the oracle; the call allocates nothing beyond its output (the codes are
    widened inside the kernel, not into per-sequence bf16 copies)."""
    import random
    from oracle.attention_ref import varlen_prefill_ref
    rng = random.Random(77 + G)
    g = torch.Generator().manual_seed(77 + G)
    Hk, D, B = 8, 128, 16
    Lq = [1, 1, 300, 1, 64, 1]
    Lk = [9000, 4000, 300 + 2000, 17, 64, 1]
    width = max((k + B - 1) // B for k in Lk)
    n_blocks = sum((k + B - 1) // B for k in Lk) + 5
    free = list(range(n_blocks))
    rng.shuffle(free)
    bt = torch.full((len(Lk), width), -1, dtype=torch.int32)
    for i, k in enumerate(Lk):
        nb = (k + B - 1) // B
        bt[i, :nb] = torch.tensor([free.pop() for _ in range(nb)], dtype=torch.int32)
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    kq, vq = fp8_ref.fp8_quantize_ref(kc, 0.5), fp8_ref.fp8_quantize_ref(vc, 0.25)
    cq = torch.tensor([0] + torch.tensor(Lq).cumsum(0).tolist(), dtype=torch.int32)
    ck = torch.tensor([0] + torch.tensor(Lk).cumsum(0).tolist(), dtype=torch.int32)
    q = torch.randn(int(cq[-1]), Hk * G, D, generator=g).to(torch.bfloat16)
    args = [x.to(dev) for x in (q, kq, vq, cq, ck, bt)]
    out = torch.empty(int(cq[-1]), Hk * G, D, dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated(dev)
    torch.cuda.reset_peak_memory_stats(dev)
    nkv.varlen_prefill(args[0], args[1].view(torch.float8_e4m3fn),
                       args[2].view(torch.float8_e4m3fn), args[3], args[4], max(Lq), D ** -0.5,
                       block_tables=args[5], out=out, max_seqlen_k=max(Lk), k_scale=0.5,
                       v_scale=0.25)
    torch.cuda.synchronize()
    assert torch.cuda.max_memory_allocated(dev) - before < 1 << 20
    kf = kq.view(torch.float8_e4m3fn).float() * 0.5
    vf = vq.view(torch.float8_e4m3fn).float() * 0.25
    ref = varlen_prefill_ref(q.float(), kf, vf, cq, ck, D ** -0.5, block_tables=bt)
    assert (out.float().cpu() - ref).abs().max().item() <= 2e-2


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float8_e4m3fn])
def test_pool_sizing_follows_the_reference_formula(nkv, dev, dtype):
    """blocks = (total * utilization - used - peak + current) // block bytes
    (model_runner.py:133-145); fp8 blocks are half the bytes. Sized to ~2 GiB."""
    torch.cuda.synchronize()
    free, total = torch.cuda.mem_get_info(dev)
    stats = torch.cuda.memory_stats(dev)
    used, peak = total - free, stats["allocated_bytes.all.peak"]
    cur = stats["allocated_bytes.all.current"]
    util = (used + peak - cur + 2 * 2 ** 30) / total
    L, Hk, D, B = 4, 8, 128, 256
    block_bytes = 2 * L * B * Hk * D * (1 if dtype == torch.float8_e4m3fn else 2)
    expect = int(total * util - used - peak + cur) // block_bytes
    pool = kvc.KVCachePool(L, Hk, D, B, dtype=dtype, gpu_memory_utilization=util, device=dev)
    assert pool.block_bytes == block_bytes
    assert abs(pool.num_blocks - expect) <= 1  # the allocator's own bookkeeping may move
    assert pool.kv_cache.shape == (2, L, pool.num_blocks, B, Hk, D)
    del pool
    torch.cuda.empty_cache()


@pytest.mark.parametrize("W,Hq,Hk", [(4, 32, 8), (4, 32, 4), (6, 32, 8), (4, 64, 2)])
@pytest.mark.parametrize("agg", ["all", "group"])
def test_compress_step_over_fp8_pool(nkv, dev, agg, W, Hq, Hk):
    """Compression on an fp8 pool: importance within rtol 1e-4 of the oracle's fp32 SnapKV on
    the fp32-dequantized window, kept sets bit-exact given those scores, and the 1-byte rows
    compacted bit-exactly; -1 padding in seq_idx skipped. Windows of 4 blocks take the fused
    kernels, 6 blocks (1536 tokens) and GQA groups above 16 (64 over 2) the general path."""
    from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                     get_tail_window_and_tail_slots_ref, select_topk_ref,
                                     snapkv_importance_ref)
    KEEP, ks = 2 * 256 + 1, 0.5
    wl = wl_mod.compress_workload(32, Hq, Hk, 1500, 4096, 6, 4, selected_only=True)
    kq = fp8_ref.fp8_quantize_ref(wl["k_cache"], ks)
    vq = fp8_ref.fp8_quantize_ref(wl["v_cache"], 2.0)
    kg = kq.to(dev).view(torch.float8_e4m3fn)
    vg = vq.to(dev).view(torch.float8_e4m3fn)
    sel = wl["seq_idx"]
    seq_idx = torch.tensor(sel[:3] + [-1] + sel[3:], dtype=torch.int32, device=dev)
    base = wl["context_lens"].to(dev)
    ctx = base.clone()
    keep, imp = cu.compress_step(wl["q"].to(dev), kg, vg, wl["block_tables"].to(dev), base, ctx,
                                 seq_idx, W, KEEP, 128 ** -0.5, agg, k_scale=ks)
    torch.cuda.synchronize()
    real = [i for i in range(seq_idx.numel()) if i != 3]
    imp, keep = imp.cpu()[real], keep.cpu()[real]
    # importance against the oracle on the fp32-dequantized K
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(wl["block_tables"], wl["context_lens"], st,
                                                   256, W)
    kf = kq.view(torch.float8_e4m3fn).float() * ks
    k_sub, _ = gather_kv_by_slots_ref(kf, kf, slots)
    ref_imp = snapkv_importance_ref(wl["q"].index_select(0, st).unsqueeze(2), k_sub, 1, "fp32",
                                    agg)
    assert torch.allclose(imp, ref_imp, rtol=1e-4, atol=1e-7)
    assert torch.equal(keep[..., 1:-1].long(), select_topk_ref(imp, KEEP - 2))
    # compaction of the codes, given the GPU's kept positions
    kc, vc, ctx_ref = kq.clone(), vq.clone(), wl["context_lens"].clone()
    compress_compact_ref(None, kc, vc, wl["block_tables"], wl["context_lens"], ctx_ref, sel, 256,
                         W, 2, 1, 0, 2, keep_idx=keep.long())
    assert torch.equal(kg.view(torch.uint8).cpu(), kc) and torch.equal(vg.view(torch.uint8).cpu(), vc)
    assert torch.equal(ctx.cpu(), ctx_ref)
