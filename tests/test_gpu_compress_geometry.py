"""Compression-step geometries beyond the reference defaults, on the GPU.

* Where a sequence's tail does not fit after the last kept token in that token's block
  (keep_tokens % B + tail > B: keep_extra_tokens = 0, or a large extra), the kernels put
  tail row u at logical position keep_tokens + u; the reference's physical slot
  slot(keep_tokens - 1) + 1 + u (compress_utils.py:210-231) would be in an unrelated block.
  Checked against the oracle (which places them the same way) and by reading the compacted
  sequence back through its block table: prefix, the kept window rows in order, the tail.
* More kept + tail rows than one read-then-write round holds: keep_blocks = 3 at B = 256
  (fused kernels, two rounds), and B = 512 with the default keep 2*512 + 1 (general path,
  up to 1536 rows).
* A selected sequence that cannot be compressed is left unchanged and its event row is
  marked skipped (n_freed = -1); the host then changes nothing for it.
"""
import importlib
import random

import pytest
import torch

from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)

pytestmark = pytest.mark.gpu
D = 128
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")


def _case(seed, B, W, lens, Hk=4, G=2):
    rng = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    width = max((n + B - 1) // B for n in lens) + 1
    n_blocks = sum((n + B - 1) // B for n in lens) + 3
    free = list(range(n_blocks))
    rng.shuffle(free)
    rows = []
    for n in lens:
        nb = (n + B - 1) // B
        rows.append([free.pop() for _ in range(nb)] + [-1] * (width - nb))
    bt = torch.tensor(rows, dtype=torch.int32)
    kc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(n_blocks, B, Hk, D, generator=g).to(torch.bfloat16)
    q = torch.randn(len(lens), Hk * G, D, generator=g).to(torch.bfloat16)
    return q, kc, vc, bt, torch.tensor(lens, dtype=torch.int32)


def _rows(cache, bt_row, n, B):
    t = torch.arange(n)
    return cache[bt_row.long()[t // B], t % B]


def _run_and_check(nkv, dev, q, kc, vc, bt, lens, sel, B, W, keep_blocks, extra, agg):
    keep = keep_blocks * B + extra
    kg, vg = kc.to(dev), vc.to(dev)
    base = lens.to(dev)
    ctx = base.clone()
    seq_idx = torch.tensor(sel, dtype=torch.int32, device=dev)
    keep_idx, imp = cu.compress_step(q.to(dev), kg, vg, bt.to(dev), base, ctx, seq_idx, W, keep,
                                     D ** -0.5, agg)
    torch.cuda.synchronize()
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt, lens, st, B, W)
    k_sub, _ = gather_kv_by_slots_ref(kc, vc, slots)
    ref_imp = snapkv_importance_ref(q.index_select(0, st).unsqueeze(2), k_sub, 1, "fp32", agg)
    assert torch.allclose(imp.cpu(), ref_imp, rtol=1e-4, atol=1e-7)
    keep_idx = keep_idx.cpu().long()
    assert torch.equal(keep_idx[..., 1:-1], select_topk_ref(imp.cpu(), keep - 2))
    # oracle compaction given the same kept positions: bit-exact caches and lengths
    kr, vr, ctx_ref = kc.clone(), vc.clone(), lens.clone()
    ok, _, _ = compress_compact_ref(None, kr, vr, bt, lens, ctx_ref, sel, B, W, keep_blocks,
                                    extra, 0, 2, keep_idx=keep_idx)
    assert ok
    kgc, vgc = kg.cpu(), vg.cpu()
    assert torch.equal(kgc, kr) and torch.equal(vgc, vr)
    assert torch.equal(ctx.cpu(), ctx_ref)
    # the compacted sequence read through its table: prefix, kept window rows, tail
    for r, s in enumerate(sel):
        n, new_n = int(lens[s]), int(ctx_ref[s])
        w0 = (n // B - W) * B
        for cache, new in ((kc, kgc), (vc, vgc)):
            old_rows = _rows(cache, bt[s], n, B)
            got = _rows(new, bt[s], new_n, B)
            assert torch.equal(got[:w0], old_rows[:w0])
            for h in range(cache.size(2)):
                ki = keep_idx[r, 0 if keep_idx.size(1) == 1 else h]
                assert torch.equal(got[w0:w0 + keep, h], old_rows[w0 + ki, h])
            assert torch.equal(got[w0 + keep:new_n], old_rows[w0 + W * B:n])
    return kg, vg, ctx


@pytest.mark.parametrize("agg", ["all", "group"])
@pytest.mark.parametrize("keep_blocks,extra", [(2, 0), (2, 200), (1, 255), (3, 0)])
def test_tail_rows_at_logical_positions(nkv, dev, agg, keep_blocks, extra):
    """Tails that cross into the next window block after the kept tokens (all three
    window blocks of a W = 4 window at B = 256; keep_blocks = 3 also takes a second
    read-then-write round in the fused kernel)."""
    B, W = 256, 4
    lens = [W * B + 17, W * B + 250, 6 * B + 100, 5 * B, 7 * B + 254, 4 * B + 1]
    q, kc, vc, bt, lt = _case(7 + keep_blocks * 31 + extra, B, W, lens)
    print(f"keep_blocks={keep_blocks} extra={extra} agg={agg}", flush=True)
    _run_and_check(nkv, dev, q, kc, vc, bt, lt, [0, 1, 2, 3, 4, 5], B, W, keep_blocks, extra,
                   agg)


@pytest.mark.parametrize("agg", ["all", "group"])
def test_block_size_512(nkv, dev, agg):
    """B = 512, W = 4 (a 2048-token window: the general path), keep 2*512 + 1: up to 1536
    kept + tail rows per (sequence, KV head), two rounds of the compaction kernel."""
    B, W = 512, 4
    lens = [W * B + 511 - 1, W * B + 3, 5 * B + 300]
    q, kc, vc, bt, lt = _case(512, B, W, lens, Hk=2, G=4)
    _run_and_check(nkv, dev, q, kc, vc, bt, lt, [0, 1, 2], B, W, 2, 1, agg)


def test_skipped_rows_marked(nkv, dev):
    """A selected sequence with fewer than W full blocks: caches and length untouched, the
    event row says n_freed = -1, and the decoded event is flagged skipped."""
    B, W = 256, 4
    lens = [W * B + 40, 3 * B + 17, 5 * B + 2]
    q, kc, vc, bt, lt = _case(99, B, W, lens)
    kg, vg = kc.to(dev), vc.to(dev)
    btg, base = bt.to(dev), lt.to(dev)
    ctx = base.clone()
    sel = torch.tensor([0, 1, 2], dtype=torch.int32, device=dev)
    cu.compress_step(q.to(dev), kg, vg, btg, base, ctx, sel, W, 2 * B + 1, D ** -0.5, "all")
    events = torch.empty(3, 4 + bt.size(1), dtype=torch.int32, device=dev)
    cu.compress_finalize(btg, base, sel, 2 * B + 1, B, W, events)
    torch.cuda.synchronize()
    ev = events.cpu()
    assert ev[1, 0] == 1 and ev[1, 1] == lens[1] and ev[1, 3] == -1
    assert int(ctx[1]) == lens[1]
    assert torch.equal(btg.cpu()[1], bt[1])  # its table is not rewritten
    for b in bt[1].tolist():
        if b >= 0:
            assert torch.equal(kg[b].cpu(), kc[b]) and torch.equal(vg[b].cpu(), vc[b])
    dicts = cu.events_to_dicts(events, 0)
    assert [d.get("skipped", False) for d in dicts] == [False, True, False]
    assert ev[0, 3] >= 1 and ev[2, 3] >= 1
