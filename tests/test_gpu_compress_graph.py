"""Device-side compression scheduling and the graph-captured compression step.

* nkv_compress_schedule vs the schedule oracle (model_runner.py:300-332): bit-exact
  selections, both policies, firing only on every period-th step.
* A -1 padded seq_idx gives the same caches, lengths and events as the unpadded one.
* A decode step with compression (device selection, store, compaction, decode, finalize for
  3 layers) captured in a HIP graph and replayed over consecutive steps equals the eager
  step with host selection, bitwise, at every step; the host applies the device events.
"""
import importlib
import random
from types import SimpleNamespace

import pytest
import torch

from oracle.compress_ref import compress_schedule_ref

pytestmark = pytest.mark.gpu
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
hooks = importlib.import_module("nanokv-llm_amd.engine.compress_hooks")
B, W = 256, 4


@pytest.mark.parametrize("policy", ["first", "longest"])
@pytest.mark.parametrize("bs,topk", [(1, 1), (37, 5), (500, 20), (1024, 64), (64, 64),
                                     (1025, 20), (200, 65), (3000, 64)])
def test_schedule_kernel_matches_oracle(dev, policy, bs, topk):
    rng = random.Random(bs * 3 + topk)
    counter_d = torch.zeros(1, dtype=torch.int32, device=dev)
    seq_idx = torch.empty(topk, dtype=torch.int32, device=dev)
    n_sel = torch.empty(1, dtype=torch.int32, device=dev)
    base = torch.empty(bs, dtype=torch.int32, device=dev)
    counter = 0
    for _ in range(4):
        lens = [rng.randrange(1, 20 * B) for _ in range(bs)]
        lens = [(n // B) * B + B - 1 if rng.random() < 0.1 else n for n in lens]
        lens = [4000 if rng.random() < 0.1 else n for n in lens]  # ties for "longest"
        tails = [rng.randrange(0, 2 * W * B) for _ in range(bs)]
        ctx = torch.tensor(lens, dtype=torch.int32, device=dev)
        cu.compress_schedule(ctx, torch.tensor(tails, dtype=torch.int32, device=dev), B, W, topk,
                             2, counter_d, seq_idx, n_sel, base, policy=policy)
        counter, sel, fired = compress_schedule_ref(lens, tails, B, W, topk, counter, 2, policy)
        assert int(counter_d) == counter
        assert seq_idx.cpu().tolist() == sel + [-1] * (topk - len(sel)), fired
        assert int(n_sel) == len(sel)
        assert torch.equal(base, ctx)


def _state(seed, bs, Hq, Hk, D, n_blocks, max_blocks):
    g = torch.Generator().manual_seed(seed)
    lens = (torch.randint(5, 12, (bs,), generator=g) * B
            + torch.randint(0, B - 8, (bs,), generator=g)).tolist()
    tails = [n if i % 3 else 100 for i, n in enumerate(lens)]  # every third not eligible
    perm = torch.randperm(n_blocks, generator=g).tolist()
    tables = [perm[i * max_blocks:(i * max_blocks) + (n + B - 1) // B] for i, n in enumerate(lens)]
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    return g, lens, tails, tables, kc, vc


def _bt(tables, width):
    return torch.tensor([t + [-1] * (width - len(t)) for t in tables], dtype=torch.int32)


def test_padded_selection_equals_unpadded(dev):
    bs, Hq, Hk, D = 8, 32, 8, 128
    g, lens, tails, tables, kc, vc = _state(30, bs, Hq, Hk, D, 96, 12)
    q = torch.randn(bs, Hq, D, generator=g).to(torch.bfloat16).to(dev)
    bt = _bt(tables, 12).to(dev)
    base = torch.tensor(lens, dtype=torch.int32, device=dev)
    outs = []
    for sel in ([1, 4], [-1, 1, -1, 4, -1]):
        k2, v2, ctx = kc.to(dev), vc.to(dev), base.clone()
        seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
        cu.compress_step(q, k2, v2, bt, base, ctx, seq_idx, W, 2 * B + 1, D ** -0.5, "group")
        ev = torch.empty(len(sel), 4 + 12, dtype=torch.int32, device=dev)
        bt2 = bt.clone()
        cu.compress_finalize(bt2, base, seq_idx, 2 * B + 1, B, W, ev)
        rows = [r for r in ev.cpu().tolist() if r[0] >= 0]
        pads = [r for r in ev.cpu().tolist() if r[0] < 0]
        assert all(r[:4] == [-1, 0, 0, 0] and set(r[4:]) == {-1} for r in pads)
        outs.append((k2.cpu(), v2.cpu(), ctx.cpu(), bt2.cpu(), rows))
    a, b = outs
    assert all(torch.equal(x, y) for x, y in zip(a[:4], b[:4])) and a[4] == b[4]


def test_graph_captured_compression_step(dev):
    nkv = importlib.import_module("nanokv-llm_amd")
    bs, Hq, Hk, D, L, MB, NB = 12, 32, 8, 128, 3, 16, 12 * 16
    cfg = SimpleNamespace(kv_compress_enabled=True, kv_compress_window_blocks=W,
                          kv_compress_keep_blocks=2, kv_compress_keep_extra_tokens=1,
                          kv_compress_agg="group", kvcache_block_size=B, kv_compress_topk=3,
                          kv_compress_period=1)
    g, lens, tails, tables, kc, vc = _state(31, bs, Hq, Hk, D, NB, MB)
    keep = 2 * B + 1

    def layers(caches):
        out = []
        for k_, v_ in caches:
            a = nkv.Attention(Hq, D, D ** -0.5, Hk, cfg, L)
            a.k_cache, a.v_cache = k_, v_
            out.append(a)
        return out

    caches_g = [(kc.to(dev), vc.to(dev)) for _ in range(L)]
    caches_e = [(kc.to(dev), vc.to(dev)) for _ in range(L)]
    att_g, att_e = layers(caches_g), layers(caches_e)
    # static graph inputs
    q_s = torch.zeros(bs, Hq, D, dtype=torch.bfloat16, device=dev)
    k_s = torch.zeros(bs, Hk, D, dtype=torch.bfloat16, device=dev)
    v_s = torch.zeros_like(k_s)
    slot_s = torch.zeros(bs, dtype=torch.int32, device=dev)
    ctx_s = torch.zeros(bs, dtype=torch.int32, device=dev)
    bt_s = torch.zeros(bs, MB, dtype=torch.int32, device=dev)
    tail_s = torch.zeros(bs, dtype=torch.int32, device=dev)
    o_s = []
    dsched = hooks.DeviceCompressionScheduler(cfg, bs, dev)

    def metadata():
        slots = [tables[i][(n - 1) // B] * B + (n - 1) % B for i, n in enumerate(lens)]
        return (torch.tensor(slots, dtype=torch.int32), torch.tensor(lens, dtype=torch.int32),
                _bt(tables, MB), torch.tensor(tails, dtype=torch.int32))

    def fill_static(step_inputs):
        q, k, v = step_inputs
        sl, cl, bt, tl = metadata()
        for dst, src in ((q_s, q), (k_s, k), (v_s, v), (slot_s, sl), (ctx_s, cl), (bt_s, bt),
                         (tail_s, tl)):
            dst.copy_(src)

    def graph_body():
        nkv.set_context(True, slot_mapping=slot_s, context_lens=ctx_s, block_tables=bt_s)
        dsched.prepare(nkv.get_context(), tail_s)
        o_s.clear()
        for li, a in enumerate(att_g):
            o_s.append(a(q_s, k_s, v_s, li))

    def step_inputs():
        return (torch.randn(bs, Hq, D, generator=g).to(torch.bfloat16),
                torch.randn(bs, Hk, D, generator=g).to(torch.bfloat16),
                torch.randn(bs, Hk, D, generator=g).to(torch.bfloat16))

    graph = None
    counter = 0
    for step in range(3):
        inp = step_inputs()
        # eager step, host selection
        sl, cl, bt, tl = metadata()
        nkv.set_context(True, slot_mapping=sl.to(dev), context_lens=cl.to(dev),
                        block_tables=bt.to(dev))
        ctx = nkv.get_context()
        counter, sel, _ = compress_schedule_ref(lens, tails, B, W, 3, counter, 1)
        ctx.is_compress_step = True
        ctx.compress_selected_batch_indices = sel
        ctx.compress_base_context_lens = ctx.context_lens.clone()
        o_e = [a(inp[0].to(dev), inp[1].to(dev), inp[2].to(dev), li)
               for li, a in enumerate(att_e)]
        torch.cuda.synchronize()
        ev_e = [e for e in ctx.compression_events if e["batch_index"] >= 0]
        ctx_e = ctx.context_lens.cpu()
        # graph step: capture on the first step, replay afterwards
        fill_static(inp)
        if graph is None:
            # every kernel of the step has run eagerly above except the scheduler: run it
            # once on scratch buffers so that nothing is loaded for the first time in capture
            scratch = [torch.zeros(k, dtype=torch.int32, device=dev) for k in (1, 3, 1, bs)]
            cu.compress_schedule(ctx_s, tail_s, B, W, 3, 1, *scratch)
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph):  # recorded, not run
                graph_body()
            events_dev = nkv.get_context().compression_events_device
        graph.replay()
        torch.cuda.synchronize()
        for (kg, vg), (ke, ve) in zip(caches_g, caches_e):
            assert torch.equal(kg, ke) and torch.equal(vg, ve), f"step {step}: caches differ"
        for og, oe in zip(o_s, o_e):
            assert torch.equal(og, oe), f"step {step}: decode outputs differ"
        assert torch.equal(ctx_s.cpu(), ctx_e)
        evs = [e for e in cu.events_to_dicts(events_dev, L - 1) if e["batch_index"] >= 0]
        assert [(e["batch_index"], e["new_context_len"], e["keep_blocks"], e["freed_block_ids"])
                for e in evs] == [(e["batch_index"], e["new_context_len"], e["keep_blocks"],
                                   e["freed_block_ids"]) for e in ev_e]
        assert [e["batch_index"] for e in evs] == sel and sel, f"step {step}: selection"
        # host bookkeeping for the next step: compressed lengths, one more token each
        for e in evs:
            i = e["batch_index"]
            lens[i] = e["new_context_len"]
            tails[i] = 0
            tables[i] = tables[i][:e["keep_blocks"]]
        for i in range(bs):
            lens[i] += 1
            tails[i] += 1
            if (lens[i] + B - 1) // B > len(tables[i]):
                raise AssertionError("test lengths were chosen to need no new block")
    nkv.reset_context()
