"""Seeded random sweeps of small configurations against the oracle.

Each case draws its own geometry: block sizes 16-256 (compression 64-512), 1-8 KV heads,
GQA groups 1-8 and 16, ragged contexts including empty and one-token ones,
tables padded with -1 or 0, and padding entries in the compression selection; head_dim 128,
with extra cases at 64 and 256. Tolerances
are the suite's: 2e-2 max abs error for bf16 attention outputs against the fp32 oracle,
bit-exact integer work (cache rows, lengths, kept indices given the scores) and importance
within rtol 1e-4.
"""
import importlib
import random

import pytest
import torch

from oracle.attention_ref import paged_decode_ref, store_kvcache_ref, varlen_prefill_ref
from oracle.compress_ref import (compress_compact_ref, gather_kv_by_slots_ref,
                                 get_tail_window_and_tail_slots_ref, select_topk_ref,
                                 snapkv_importance_ref)

pytestmark = pytest.mark.gpu
TOL = 2e-2
cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")


def _cases(n128, n_other, base=0):
    """(case, head_dim): n128 cases at 128, then n_other each at 64 and 256."""
    return ([(c, 128) for c in range(n128)] +
            [(n128 + i, 64) for i in range(n_other)] +
            [(n128 + n_other + i, 256) for i in range(n_other)])


def _randn(shape, g, scale=1.0):
    return (torch.randn(shape, generator=g) * scale).to(torch.bfloat16)


def _tables(rng, lens, B, n_blocks, width, pad):
    """Distinct random physical blocks per sequence, rows padded with `pad`."""
    free = list(range(n_blocks))
    rng.shuffle(free)
    rows = []
    for n in lens:
        nb = (n + B - 1) // B
        rows.append([free.pop() for _ in range(nb)] + [pad] * (width - nb))
    return torch.tensor(rows, dtype=torch.int32).reshape(len(lens), width)


@pytest.mark.parametrize("case,D", _cases(24, 6))
def test_decode_sweep(nkv, dev, case, D):
    rng = random.Random(1000 + case)
    g = torch.Generator().manual_seed(1000 + case)
    B = rng.choice([16, 32, 64, 128, 256])
    Hk = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16])
    bs = rng.randrange(1, 70)
    top = rng.choice([40, 600, 3000])
    lens = [rng.choice([0, 1, rng.randrange(1, top + 1), rng.randrange(1, top + 1)])
            for _ in range(bs)]
    width = max(1, max((n + B - 1) // B for n in lens)) + rng.randrange(0, 3)
    n_blocks = sum((n + B - 1) // B for n in lens) + 4
    bt = _tables(rng, lens, B, n_blocks, width, rng.choice([-1, 0]))
    kc, vc = _randn((n_blocks, B, Hk, D), g), _randn((n_blocks, B, Hk, D), g)
    q = _randn((bs, Hk * G, D), g)
    ctx = torch.tensor(lens, dtype=torch.int32)
    print(f"decode case {case}: D={D} B={B} Hk={Hk} G={G} bs={bs} max_len={max(lens)}",
          flush=True)
    out = nkv.paged_decode(q.to(dev), kc.to(dev), vc.to(dev), ctx.to(dev), bt.to(dev), D ** -0.5)
    torch.cuda.synchronize()
    ref = paged_decode_ref(q.float(), kc, vc, ctx, bt, D ** -0.5)
    assert (out.float().cpu() - ref).abs().max().item() <= TOL


@pytest.mark.parametrize("case,D", _cases(16, 6))
def test_prefill_sweep(nkv, dev, case, D):
    rng = random.Random(2000 + case)
    g = torch.Generator().manual_seed(2000 + case)
    paged = case % 4 != 3
    B = rng.choice([16, 32, 64, 128, 256])
    Hk = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 3, 4, 5, 6, 8, 16])
    n = rng.randrange(1, 7)
    Lq, Lk = [], []
    for _ in range(n):
        lq = rng.choice([1, rng.randrange(1, 300), rng.randrange(1, 700)])
        pre = rng.choice([0, 0, rng.randrange(0, 900)])
        Lq.append(lq)
        Lk.append(lq + pre)
    cq = torch.tensor([0] + torch.tensor(Lq).cumsum(0).tolist(), dtype=torch.int32)
    ck = torch.tensor([0] + torch.tensor(Lk).cumsum(0).tolist(), dtype=torch.int32)
    q = _randn((int(cq[-1]), Hk * G, D), g)
    print(f"prefill case {case}: D={D} paged={paged} B={B} Hk={Hk} G={G} Lq={Lq} Lk={Lk}",
          flush=True)
    if paged:
        n_blocks = sum((k + B - 1) // B for k in Lk) + 3
        width = max((k + B - 1) // B for k in Lk) + rng.randrange(0, 2)
        bt = _tables(rng, Lk, B, n_blocks, width, -1)
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


@pytest.mark.parametrize("case,D", _cases(8, 2))
def test_store_sweep(nkv, dev, case, D):
    rng = random.Random(3000 + case)
    g = torch.Generator().manual_seed(3000 + case)
    B = rng.choice([16, 64, 256])
    Hk = rng.choice([1, 2, 4, 8])
    n_blocks = rng.randrange(2, 40)
    N = rng.randrange(1, 3000)
    slots = rng.sample(range(n_blocks * B), min(N, n_blocks * B))
    slots += [-1] * (N - len(slots))
    rng.shuffle(slots)
    slots = [-1 if rng.random() < 0.1 else s for s in slots]
    extra = rng.choice([0, 8, 3 * Hk * D])  # key/value rows inside a wider projection
    key = _randn((N, Hk * D + extra), g)[:, :Hk * D].reshape(N, Hk, D)
    value = _randn((N, Hk * D + extra), g)[:, :Hk * D].reshape(N, Hk, D)
    kc, vc = _randn((n_blocks, B, Hk, D), g), _randn((n_blocks, B, Hk, D), g)
    sm = torch.tensor(slots, dtype=torch.int32)
    print(f"store case {case}: D={D} B={B} Hk={Hk} N={N} row_stride={key.stride(0)}",
          flush=True)
    kg, vg = kc.to(dev), vc.to(dev)
    nkv.store_kvcache(key.to(dev), value.to(dev), kg, vg, sm.to(dev))
    torch.cuda.synchronize()
    store_kvcache_ref(key, value, kc, vc, sm)
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)


@pytest.mark.parametrize("case,D", _cases(12, 3))
def test_compress_step_sweep(nkv, dev, case, D):
    rng = random.Random(4000 + case)
    g = torch.Generator().manual_seed(4000 + case)
    # head_dim 64 / 256 take the general path, whose scoring reads 256-key chunks of one block
    B = rng.choice([64, 128, 256]) if D == 128 else 256
    W = rng.choice([2, 3, 4]) if B == 256 else rng.choice([2, 4])
    # any keep (one or more read-then-write rounds, tails at logical positions); the last
    # case has a window over 1024 tokens: the general path (score, importance, top-k and a
    # compaction of up to 1323 rows in two rounds)
    choices = [(kb, ex) for kb in range(1, W) for ex in (0, 1, B // 2)]
    keep_blocks, extra = rng.choice(choices)
    if case == 11:
        B, W, keep_blocks, extra = 512, 3, 1, 300
    keep = keep_blocks * B + extra
    Hk = rng.choice([1, 2, 4, 8])
    G = rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16])
    agg = rng.choice(["all", "group"])
    bs = rng.randrange(2, 24)
    # eligible lengths: at least W full blocks, tail != B - 1
    lens = []
    for _ in range(bs):
        n = rng.randrange(W * B, (W + 5) * B)
        lens.append(n - 1 if n % B == B - 1 else n)
    width = max((n + B - 1) // B for n in lens) + rng.randrange(0, 2)
    n_blocks = sum((n + B - 1) // B for n in lens) + 2
    bt = _tables(rng, lens, B, n_blocks, width, -1)
    kc, vc = _randn((n_blocks, B, Hk, D), g), _randn((n_blocks, B, Hk, D), g)
    q = _randn((bs, Hk * G, D), g)
    sel = sorted(rng.sample(range(bs), rng.randrange(1, min(bs, 8) + 1)))
    padded = list(sel)
    if case % 3 == 0:
        padded.insert(rng.randrange(0, len(padded) + 1), -1)
    print(f"compress case {case}: D={D} B={B} W={W} keep={keep} Hk={Hk} G={G} agg={agg} "
          f"sel={padded} last_layer={case % 2 == 1}", flush=True)
    base = torch.tensor(lens, dtype=torch.int32)
    kg, vg, ctx = kc.to(dev), vc.to(dev), base.clone().to(dev)
    seq_idx = torch.tensor(padded, dtype=torch.int32, device=dev)
    # odd cases: the last layer's step, with the finalize's events, table and slot rewrite
    last = case % 2 == 1
    btg = bt.to(dev)
    events = torch.full((len(padded), 4 + width), 77, dtype=torch.int32, device=dev)
    slot_map = torch.arange(bs, dtype=torch.int32, device=dev) * 5 + 3
    fin = dict(events=events, rewrite_tables=True, slot_mapping=slot_map) if last else {}
    keep_idx, imp = cu.compress_step(q.to(dev), kg, vg, btg, base.to(dev), ctx, seq_idx, W,
                                     keep, D ** -0.5, agg, **fin)
    torch.cuda.synchronize()
    real = [i for i, s in enumerate(padded) if s >= 0]
    imp, keep_idx = imp.cpu()[real], keep_idx.cpu()[real]
    st = torch.tensor(sel)
    slots, *_ = get_tail_window_and_tail_slots_ref(bt, base, st, B, W)
    k_sub, _ = gather_kv_by_slots_ref(kc, vc, slots)
    ref_imp = snapkv_importance_ref(q.index_select(0, st).unsqueeze(2), k_sub, 1, "fp32", agg)
    assert torch.allclose(imp, ref_imp, rtol=1e-4, atol=1e-7)
    assert torch.equal(keep_idx[..., 1:-1].long(), select_topk_ref(imp, keep - 2))
    ctx_ref = base.clone()
    _, _, ev_ref = compress_compact_ref(None, kc, vc, bt, base, ctx_ref, sel, B, W, keep_blocks,
                                        extra, 0, 1 if last else 2, keep_idx=keep_idx.long())
    assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    assert torch.equal(ctx.cpu(), ctx_ref)
    if last:  # events (padding rows skipped), freed table entries -1, the next token's slot
        assert cu.events_to_dicts(events, 0) == ev_ref
        bt_exp = bt.clone()
        slot_exp = torch.arange(bs, dtype=torch.int32) * 5 + 3
        for ev in ev_ref:
            i, n = ev["batch_index"], ev["new_context_len"]
            bt_exp[i, ev["keep_blocks"]:] = -1
            slot_exp[i] = -1 if n % B == 0 else int(bt[i, n // B]) * B + n % B
        assert torch.equal(btg.cpu(), bt_exp) and torch.equal(slot_map.cpu(), slot_exp)
