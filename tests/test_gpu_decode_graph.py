"""The decode branch of Attention.forward (store the new token, then attend) captured in a
HIP graph and replayed, as the reference's model runner captures decode steps
(nanokvllm/engine/model_runner.py:400-441).

The graph is captured once over static tensors (q, k, v, slot mapping, context lengths,
block tables, as the runner's graph buffers); each of several decode steps writes that
step's inputs into them, replays, and is compared bit for bit with the same step run
eagerly on a second copy of the caches: the output and both caches. Eager work and a
synchronisation run between the replays. Both pools: bf16 and fp8 (E4M3FN).
"""
import importlib
from types import SimpleNamespace

import pytest
import torch

pytestmark = pytest.mark.gpu
kvc = importlib.import_module("nanokv-llm_amd.layers.kv_cache")

BS, HQ, HK, D, B, STEPS = 6, 32, 8, 128, 256, 4


def _state(seed):
    g = torch.Generator().manual_seed(seed)
    ctx0 = torch.randint(200, 1500, (BS,), generator=g, dtype=torch.int64)
    need = [(int(c) + STEPS + B - 1) // B for c in ctx0]
    n_blocks = sum(need) + 4
    perm = torch.randperm(n_blocks, generator=g).tolist()
    width = max(need) + 1  # one padding column, as graph buffers pad
    rows, o = [], 0
    for n in need:
        rows.append(perm[o:o + n] + [0] * (width - n))
        o += n
    bt = torch.tensor(rows, dtype=torch.int32)
    kc = torch.randn(n_blocks, B, HK, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, HK, D, generator=g).to(torch.bfloat16)
    steps = []
    for i in range(STEPS):
        ctx = ctx0 + i + 1  # context lengths include the token stored this step
        pos = ctx - 1
        slots = (bt.to(torch.int64)[torch.arange(BS), pos // B] * B + pos % B).to(torch.int32)
        steps.append(dict(q=torch.randn(BS, HQ, D, generator=g).to(torch.bfloat16),
                          k=torch.randn(BS, HK, D, generator=g).to(torch.bfloat16),
                          v=torch.randn(BS, HK, D, generator=g).to(torch.bfloat16),
                          ctx=ctx.to(torch.int32), slots=slots))
    return kc, vc, bt, steps


@pytest.mark.parametrize("fp8", [False, True])
def test_decode_step_replayed_from_a_graph(nkv, dev, fp8):
    kc, vc, bt, steps = _state(21 + int(fp8))
    cfg = SimpleNamespace(kv_compress_enabled=False)

    def layer(k_cache, v_cache):
        a = nkv.Attention(HQ, D, D ** -0.5, HK, cfg, 1)
        a.k_cache, a.v_cache = k_cache, v_cache
        return a

    def pool():
        k, v = kc.to(dev), vc.to(dev)
        return (kvc.fp8_quantize(k), kvc.fp8_quantize(v)) if fp8 else (k, v)

    gk, gv = pool()
    ek, ev = pool()
    g_attn, e_attn = layer(gk, gv), layer(ek, ev)
    # static graph inputs
    sq = torch.empty(BS, HQ, D, dtype=torch.bfloat16, device=dev)
    sk = torch.empty(BS, HK, D, dtype=torch.bfloat16, device=dev)
    sv = torch.empty(BS, HK, D, dtype=torch.bfloat16, device=dev)
    s_slots = torch.empty(BS, dtype=torch.int32, device=dev)
    s_ctx = torch.empty(BS, dtype=torch.int32, device=dev)
    s_bt = bt.to(dev)

    def load(st):
        sq.copy_(st["q"]), sk.copy_(st["k"]), sv.copy_(st["v"])
        s_slots.copy_(st["slots"]), s_ctx.copy_(st["ctx"])

    def body():
        return g_attn(sq, sk, sv, 0)

    nkv.set_context(True, slot_mapping=s_slots, context_lens=s_ctx, block_tables=s_bt)
    try:
        load(steps[0])
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up (stores step 0's token, as the replay will)
            body()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = body()
        for i, st in enumerate(steps):
            load(st)
            graph.replay()
            torch.cuda.synchronize()
            got = out.clone()
            # the same step eagerly on the second pool, then unrelated eager work
            nkv.set_context(True, slot_mapping=st["slots"].to(dev),
                            context_lens=st["ctx"].to(dev), block_tables=s_bt)
            ref = e_attn(st["q"].to(dev), st["k"].to(dev), st["v"].to(dev), 0)
            nkv.set_context(True, slot_mapping=s_slots, context_lens=s_ctx, block_tables=s_bt)
            torch.randn(1 << 20, device=dev).sum().item()
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f"step {i}: replay differs from the eager step"
            assert torch.equal(gk.view(torch.uint8) if fp8 else gk,
                               ek.view(torch.uint8) if fp8 else ek), f"step {i}: K cache"
            assert torch.equal(gv.view(torch.uint8) if fp8 else gv,
                               ev.view(torch.uint8) if fp8 else ev), f"step {i}: V cache"
    finally:
        nkv.reset_context()
