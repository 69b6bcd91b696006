"""Parity at the benchmarked sizes (the workloads bench.py times, same seeds).

* Decode at Qwen3-8B geometry, batch 64 (seed 2): the new token stored, then every one of the
  64 sequences against the fp32 oracle (max abs err <= 2e-2).
* The compression step at batch 500 (seed 3: the 20 longest, W 4, keep 513), both
  aggregations: importance within rtol 1e-4 of the fp32 oracle, kept sets exact given the
  scores, caches, lengths, events, block tables and slot maps bit-exact. The same for the
  long-context state at Qwen3-32B geometry (seed 6: Hq 64 over Hk 8, the 20 longest
  eligible sequences).
* Long-context decode at Qwen3-32B geometry (seed 6: batch 500, contexts log-uniform
  [1024, 16384], 20% compressed once): 72 of the 500 sequences against the oracle.
* The same shape through a stack of Attention layers sharing one decode workspace.
"""
import importlib
from types import SimpleNamespace

import pytest
import torch

from oracle.attention_ref import paged_decode_ref
from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)

pytestmark = pytest.mark.gpu
TOL = 2e-2
wl_mod = importlib.import_module("nanokv-llm_amd.workloads")
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
attn_mod = importlib.import_module("nanokv-llm_amd.layers.attention")
kv_mod = importlib.import_module("nanokv-llm_amd.layers.kv_cache")


def _gather(bt_rows, kc, vc):
    """The blocks of some table rows copied to host, with the rows remapped onto them."""
    ids = sorted({int(x) for x in bt_rows.flatten().tolist() if x >= 0})
    remap = {b: j for j, b in enumerate(ids)}
    idx = torch.tensor(ids, device=kc.device)
    kh, vh = kc.index_select(0, idx).cpu(), vc.index_select(0, idx).cpu()
    bt2 = torch.tensor([[remap.get(int(x), -1) for x in row] for row in bt_rows.tolist()],
                       dtype=torch.int32)
    return kh, vh, bt2


def _decode_error(q, out, kc, vc, ctx, bt, scale, rows):
    """Max abs error of out[rows] against the oracle, 16 sequences at a time."""
    err = 0.0
    for i in range(0, len(rows), 16):
        r = torch.tensor(rows[i:i + 16])
        kh, vh, bt2 = _gather(bt.cpu()[r], kc, vc)
        ref = paged_decode_ref(q.cpu()[r].float(), kh, vh, ctx.cpu()[r], bt2, scale)
        err = max(err, (out.cpu()[r].float() - ref).abs().max().item())
    return err


def test_decode_qwen3_8b_all_sequences(nkv, dev):
    wl = wl_mod.decode_qwen3_8b(seed=2, device=dev)
    kc, vc = wl["k_cache"], wl["v_cache"]
    bt, slots = wl["block_tables"][0].to(dev), wl["slot_mappings"][0].to(dev)
    q, ctx = wl["q"].to(dev), wl["context_lens"].to(dev)
    nkv.store_kvcache(wl["key"].to(dev), wl["value"].to(dev), kc, vc, slots)
    out = nkv.paged_decode(q, kc, vc, ctx, bt, wl["scale"])
    torch.cuda.synchronize()
    err = _decode_error(q, out, kc, vc, ctx, bt, wl["scale"], list(range(64)))
    print(f"decode Qwen3-8B batch 64: max abs err {err:.2e}", flush=True)
    assert err <= TOL


def _check_compress_step(cw, dev, agg):
    """The compression step (compress_step + compress_finalize with the table and slot
    rewrite) on a compact copy of the state against the oracle: importance within rtol 1e-4
    of the fp32 oracle, kept sets exact given the scores, caches, lengths, events, block
    tables and slot maps bit-exact."""
    kc0, vc0 = cw["k_cache"].cpu(), cw["v_cache"].cpu()
    kg, vg = cw["k_cache"], cw["v_cache"]
    bt, lens, sel = cw["block_tables"], cw["context_lens"], cw["seq_idx"]
    bs, Hq, D = cw["q"].shape
    m = len(sel)
    print(f"compression step: batch {bs}, Hq {Hq}, Hk {kg.size(2)}, {m} sequences, agg {agg}",
          flush=True)
    btg, base = bt.to(dev), lens.to(dev)
    ctx = base.clone()
    seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
    slot_map = torch.arange(bs, dtype=torch.int32, device=dev) * 3
    keep, imp = cu.compress_step(cw["q"].to(dev), kg, vg, btg, base, ctx, seq_idx, 4, 513,
                                 D ** -0.5, agg)
    events = torch.empty(m, 4 + bt.size(1), dtype=torch.int32, device=dev)
    cu.compress_finalize(btg, base, seq_idx, 513, 256, 4, events, rewrite_tables=True,
                         slot_mapping=slot_map)
    torch.cuda.synchronize()
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt, lens, st, 256, 4)
    k_sub, _ = gather_kv_by_slots_ref(kc0, vc0, slots)
    ref_imp = snapkv_importance_ref(cw["q"].index_select(0, st).unsqueeze(2), k_sub, 1, "fp32",
                                    agg)
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    keep = keep.cpu().long()
    assert torch.equal(keep[..., 1:-1], select_topk_ref(imp.cpu(), 511))
    ctx_ref = lens.clone()
    ok, _, ev_ref = compress_compact_ref(None, kc0, vc0, bt, lens, ctx_ref, sel, 256, 4, 2, 1,
                                         0, 1, keep_idx=keep)
    assert ok
    assert torch.equal(kg.cpu(), kc0) and torch.equal(vg.cpu(), vc0)
    assert torch.equal(ctx.cpu(), ctx_ref)
    assert cu.events_to_dicts(events, 0) == ev_ref
    bt_exp = bt.clone()
    slot_exp = torch.arange(bs, dtype=torch.int32) * 3
    for ev in ev_ref:
        s, n = ev["batch_index"], ev["new_context_len"]
        bt_exp[s, ev["keep_blocks"]:] = -1
        # the next token's slot; position n opens a freed block when n % 256 == 0
        slot_exp[s] = -1 if n % 256 == 0 else int(bt[s, n // 256]) * 256 + n % 256
    assert torch.equal(btg.cpu(), bt_exp)
    assert torch.equal(slot_map.cpu(), slot_exp)


@pytest.mark.parametrize("agg", ["group", "all"])
def test_compress_step_qwen3_8b_batch_500(nkv, dev, agg):
    cw = wl_mod.compress_qwen3_8b(seed=3, device=dev, selected_only=True)
    assert len(cw["seq_idx"]) == 20 and cw["context_lens"].numel() == 500
    _check_compress_step(cw, dev, agg)


@pytest.mark.parametrize("agg", ["group", "all"])
def test_compress_step_qwen3_32b_longctx_batch_500(nkv, dev, agg):
    """The long-context state's compression step at its own geometry: Hq 64 over Hk 8
    (group 8), the 20 longest eligible sequences (15-16k tokens, 64-block tables), window
    4 blocks, keep 513."""
    cw = wl_mod.compress_qwen3_32b_longctx(seed=6, device=dev)
    assert len(cw["seq_idx"]) == 20 and cw["q"].shape == (500, 64, 128)
    assert cw["block_tables"].size(1) == 64
    _check_compress_step(cw, dev, agg)
    del cw
    torch.cuda.empty_cache()


def test_decode_qwen3_32b_batch_500(nkv, dev):
    wl = wl_mod.decode_qwen3_32b_longctx(seed=6, device=dev, n_blocks=0)
    kc, vc = wl["k_cache"], wl["v_cache"]
    bt, slots = wl["block_tables"][0].to(dev), wl["slot_mappings"][0].to(dev)
    q, ctx = wl["q"].to(dev), wl["context_lens"].to(dev)
    assert bt.size(1) == 64 and q.shape == (500, 64, 128)
    nkv.store_kvcache(wl["key"].to(dev), wl["value"].to(dev), kc, vc, slots)
    out = nkv.paged_decode(q, kc, vc, ctx, bt, wl["scale"])
    torch.cuda.synchronize()
    rows = list(range(0, 500, 7))  # 72 sequences, compressed and not
    assert any(bool(wl["compressed"][r]) for r in rows)
    err = _decode_error(q, out, kc, vc, ctx, bt, wl["scale"], rows)
    print(f"decode Qwen3-32B batch 500: max abs err {err:.2e} on {len(rows)} sequences",
          flush=True)
    assert err <= TOL
    del wl, kc, vc
    torch.cuda.empty_cache()


def test_attention_stack_qwen3_32b_batch_500(nkv, dev):
    """Three Attention layers over one KV pool at Qwen3-32B geometry, batch 500, 64-block
    tables: every layer's decode goes through the one shared workspace (no per-layer
    buffers, ~35 MB), and each layer's output matches the oracle on a sample."""
    L = 3
    wl = wl_mod.decode_qwen3_32b_longctx(seed=6, n_blocks=0, alloc_caches=False)
    bt = wl["block_tables"][0]
    ctx, slots = wl["context_lens"], wl["slot_mappings"][0]
    n_blocks = wl["n_blocks"]
    pool = kv_mod.KVCachePool(L, 8, 128, 256, num_blocks=n_blocks, device=dev)
    cfg = SimpleNamespace(kv_compress_enabled=False)
    layers = [nkv.Attention(64, 128, 128 ** -0.5, 8, cfg, L) for _ in range(L)]
    assert pool.bind(layers) == L
    used = bt[bt >= 0].to(torch.int64)
    g = torch.Generator(device=dev)
    g.manual_seed(32)
    for a in layers:  # fill the used blocks of every layer, 1 GiB at a time
        for i in range(0, used.numel(), 1024):
            ids = used[i:i + 1024].to(dev)
            shape = (ids.numel(), 256, 8, 128)
            a.k_cache[ids] = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
            a.v_cache[ids] = torch.randn(shape, generator=g, device=dev).to(torch.bfloat16)
    qs = [torch.randn(500, 64, 128, generator=g, device=dev).to(torch.bfloat16)
          for _ in range(L)]
    ks = [torch.randn(500, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    vs = [torch.randn(500, 8, 128, generator=g, device=dev).to(torch.bfloat16) for _ in range(L)]
    btg, ctxg = bt.to(dev), ctx.to(dev)
    nkv.set_context(True, slot_mapping=slots.to(dev), context_lens=ctxg, block_tables=btg)
    before = len(attn_mod._SHARED_WS)
    outs = [a(qs[i], ks[i], vs[i], i) for i, a in enumerate(layers)]
    torch.cuda.synchronize()
    nkv.reset_context()
    ws = attn_mod._SHARED_WS[torch.device(dev)]
    need = attn_mod.decode_workspace_bytes(500, 64, 64, 256)
    print(f"shared decode workspace: {ws.numel() / 1e6:.1f} MB (needs {need / 1e6:.1f} MB)",
          flush=True)
    assert len(attn_mod._SHARED_WS) <= before + 1
    assert ws.numel() >= need and need <= 100e6
    rows = list(range(3, 500, 31))  # 17 sequences
    for i, a in enumerate(layers):
        assert outs[i].shape == (500, 1, 64, 128)
        err = _decode_error(qs[i], outs[i][:, 0], a.k_cache, a.v_cache, ctxg, btg,
                            128 ** -0.5, rows)
        assert err <= TOL, f"layer {i}: max abs err {err}"
    del pool, layers
    torch.cuda.empty_cache()
