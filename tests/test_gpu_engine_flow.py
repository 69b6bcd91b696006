"""Drop-in flow on the GPU: engine hooks + Attention.forward (2 layers) through a
compression step and the decode steps after it, against the oracle on CPU copies.

Per decode step: prepare_decode_metadata -> set_context -> CompressionScheduler.prepare
-> Attention.forward per layer (store, MyCompressCompact on compress steps, decode) ->
apply_compression_events -> append. The oracle replays store_kvcache, the compaction
with the GPU's kept indices, and paged decode on the engine's block tables.
"""
import importlib
from types import SimpleNamespace

import pytest
import torch

from oracle.attention_ref import paged_decode_ref, store_kvcache_ref
from oracle.compress_ref import compress_compact_ref

pytestmark = pytest.mark.gpu
TOL = 2e-2
hooks = importlib.import_module("nanokv-llm_amd.engine.compress_hooks")
import sequence as seqmod  # noqa: E402  (test double, tests/sequence.py)
import block_manager as bmmod  # noqa: E402  (test double, tests/block_manager.py)
B, W, Hq, Hk, D, LAYERS = 256, 4, 16, 4, 128, 2


@pytest.mark.parametrize("agg", ["all", "group"])
def test_compress_then_decode(nkv, dev, agg):
    g = torch.Generator().manual_seed(77)
    cfg = SimpleNamespace(kv_compress_enabled=True, kv_compress_window_blocks=W,
                          kv_compress_keep_blocks=2, kv_compress_keep_extra_tokens=1,
                          kv_compress_agg=agg, kvcache_block_size=B, kv_compress_topk=3,
                          kv_compress_period=2)
    n_blocks = 64
    bm = bmmod.BlockManager(n_blocks, B)
    lens = [1100, 1300, 2600, 500, 1800]
    seqs = []
    for i, n in enumerate(lens):
        s = seqmod.Sequence(n, seq_id=i)
        s.tail_uncompressed_len = n
        bm.allocate(s)
        s.num_computed_tokens = n
        seqs.append(s)
    caches = [(torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16),
               torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16))
              for _ in range(LAYERS)]
    layers = []
    for kc, vc in caches:
        a = nkv.Attention(Hq, D, D ** -0.5, Hk, cfg, LAYERS)
        a.k_cache, a.v_cache = kc.to(dev), vc.to(dev)
        layers.append(a)
    sched = hooks.CompressionScheduler(cfg)
    compressed = 0
    for step in range(4):
        for s in seqs:  # this step's token is part of the context
            s.append_token()
            bm.may_append(s)
        md = hooks.prepare_decode_metadata(seqs, B, device=dev)
        nkv.set_context(True, slot_mapping=md["slot_mapping"], context_lens=md["context_lens"],
                        block_tables=md["block_tables"])
        ctx = nkv.get_context()
        sched.prepare(ctx, seqs)
        # snapshots: the last layer's finalize rewrites tables and slots in place
        bt_before = md["block_tables"].cpu()
        slots = md["slot_mapping"].cpu()
        base_lens = md["context_lens"].cpu()
        for li, attn in enumerate(layers):
            q = torch.randn(len(seqs), Hq, D, generator=g).to(torch.bfloat16)
            k = torch.randn(len(seqs), Hk, D, generator=g).to(torch.bfloat16)
            v = torch.randn(len(seqs), Hk, D, generator=g).to(torch.bfloat16)
            o = attn(q.to(dev), k.to(dev), v.to(dev), li)
            torch.cuda.synchronize()
            # oracle replay on the CPU copy of this layer's cache
            kc, vc = caches[li]
            store_kvcache_ref(k, v, kc, vc, slots)
            ctx_ref = base_lens.clone()
            sel = ctx.compress_selected_batch_indices
            if ctx.is_compress_step and sel:
                keep = ctx._nkv_compress_buffers.keep_idx.cpu().long()
                ok, _, _ = compress_compact_ref(None, kc, vc, bt_before, base_lens, ctx_ref, sel, B,
                                                W, 2, 1, li, LAYERS, keep_idx=keep)
                assert ok
            assert torch.equal(attn.k_cache.cpu(), kc), (step, li)
            assert torch.equal(attn.v_cache.cpu(), vc)
            assert torch.equal(ctx.context_lens.cpu(), ctx_ref)
            ref = paged_decode_ref(q.float(), kc, vc, ctx_ref, bt_before, D ** -0.5)
            err = (o[:, 0].float().cpu() - ref).abs().amax(dim=(1, 2))
            assert err.max().item() <= TOL, (step, li, err.tolist())
        if ctx.is_compress_step and ctx.compress_selected_batch_indices:
            compressed += len(ctx.compress_selected_batch_indices)
            evs = ctx.compression_events
            assert [e["batch_index"] for e in evs] == ctx.compress_selected_batch_indices
            hooks.apply_compression_events([seqmod.ScheduledSeq(s, 1) for s in seqs], evs, bm)
        nkv.reset_context()
    assert compressed >= 3  # step 2 compressed the first three eligible sequences
    assert len(seqs[3]) == 500 + 4  # too short to compress
