"""Pins the oracle's store / decode / prefill against independent checks (CPU).

None of these re-types the oracle's formula: they use pure-Python float64
loops, torch's scaled_dot_product_attention, and closed forms (ctx=1, equal
keys, block permutation, GQA == repeated-head MHA, chunked == one-shot).
"""
import math

import pytest
import torch
import torch.nn.functional as F

from oracle.attention_ref import (gather_paged_rows, paged_decode_ref, store_kvcache_ref,
                                  varlen_prefill_ref, varlen_prefill_rows_ref)


def _pool(nb, B, Hk, D, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(nb, B, Hk, D, generator=g), torch.randn(nb, B, Hk, D, generator=g))


# ---------------------------------------------------------------- store
def test_store_matches_slot_loop():
    g = torch.Generator().manual_seed(0)
    N, Hk, D, nb, B = 7, 2, 4, 5, 4
    key = torch.randn(N, Hk, D, generator=g)
    value = torch.randn(N, Hk, D, generator=g)
    kc, vc = torch.zeros(nb, B, Hk, D), torch.zeros(nb, B, Hk, D)
    slots = torch.tensor([3, -1, 17, 0, 19, -1, 8], dtype=torch.int32)
    exp_k, exp_v = kc.clone(), vc.clone()
    for i in range(N):
        s = int(slots[i])
        if s == -1:
            continue
        for h in range(Hk):
            for d in range(D):
                exp_k[s // B, s % B, h, d] = key[i, h, d]
                exp_v[s // B, s % B, h, d] = value[i, h, d]
    store_kvcache_ref(key, value, kc, vc, slots)
    assert torch.equal(kc, exp_k) and torch.equal(vc, exp_v)
    # every slot not named keeps its old content
    named = {int(s) for s in slots if s != -1}
    for s in range(nb * B):
        if s not in named:
            assert torch.all(kc.view(-1, Hk, D)[s] == 0)


# ---------------------------------------------------------------- decode
def _decode_loop_f64(q, kc, vc, ctx, bt, scale):
    bs, Hq, D = q.shape
    Hk = kc.size(2)
    g = Hq // Hk
    B = kc.size(1)
    out = torch.zeros(bs, Hq, D, dtype=torch.float64)
    for b in range(bs):
        for h in range(Hq):
            kh = h // g
            scores = []
            for t in range(int(ctx[b])):
                blk = int(bt[b, t // B])
                k = kc[blk, t % B, kh].double()
                scores.append(float((q[b, h].double() * k).sum()) * scale)
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            z = sum(w)
            for t in range(int(ctx[b])):
                blk = int(bt[b, t // B])
                out[b, h] += (w[t] / z) * vc[blk, t % B, kh].double()
    return out


def test_decode_matches_float64_loops():
    kc, vc = _pool(6, 4, 2, 8, 1)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(3, 4, 8, generator=g)
    bt = torch.tensor([[5, 0, -1], [2, 3, 1], [4, -1, -1]], dtype=torch.int32)
    ctx = torch.tensor([7, 10, 3], dtype=torch.int32)
    ref = paged_decode_ref(q, kc, vc, ctx, bt, 0.3)
    exp = _decode_loop_f64(q, kc, vc, ctx, bt, 0.3)
    assert torch.allclose(ref.double(), exp, atol=1e-5)


def test_decode_matches_sdpa():
    kc, vc = _pool(12, 16, 2, 32, 3)
    g = torch.Generator().manual_seed(4)
    q = torch.randn(3, 8, 32, generator=g)
    bt = torch.tensor([[11, 4, 7], [0, 1, -1], [9, 2, 3]], dtype=torch.int32)
    ctx = torch.tensor([40, 17, 48], dtype=torch.int32)
    ref = paged_decode_ref(q, kc, vc, ctx, bt, 32 ** -0.5)
    for b in range(3):
        K = gather_paged_rows(kc, bt[b], int(ctx[b])).permute(1, 0, 2)  # [Hk, n, D]
        V = gather_paged_rows(vc, bt[b], int(ctx[b])).permute(1, 0, 2)
        o = F.scaled_dot_product_attention(
            q[b].view(2, 4, 1, 32), K.unsqueeze(1).expand(2, 4, -1, 32),
            V.unsqueeze(1).expand(2, 4, -1, 32))
        assert torch.allclose(ref[b], o.reshape(8, 32), atol=1e-5)


def test_decode_closed_forms():
    kc, vc = _pool(4, 8, 2, 16, 5)
    q = torch.randn(2, 4, 16)
    bt = torch.tensor([[2, 1], [3, 0]], dtype=torch.int32)
    # ctx = 1 -> the first value row of the sequence, for every head of the group
    out = paged_decode_ref(q, kc, vc, torch.tensor([1, 1], dtype=torch.int32), bt, 1.0)
    assert torch.allclose(out[0, 0], vc[2, 0, 0]) and torch.allclose(out[0, 3], vc[2, 0, 1])
    assert torch.allclose(out[1, 2], vc[3, 0, 1])
    # equal keys -> mean of the values
    kc2 = kc.clone()
    kc2[:] = kc2[0, 0]
    out = paged_decode_ref(q, kc2, vc, torch.tensor([11, 16], dtype=torch.int32), bt, 1.0)
    V = gather_paged_rows(vc, bt[0], 11)
    assert torch.allclose(out[0, 1], V[:, 0].mean(0), atol=1e-5)
    assert torch.allclose(out[0, 2], V[:, 1].mean(0), atol=1e-5)


def test_decode_block_permutation_invariance():
    kc, vc = _pool(8, 4, 2, 8, 6)
    q = torch.randn(2, 2, 8)
    bt = torch.tensor([[0, 1, 2], [3, 4, 5]], dtype=torch.int32)
    ctx = torch.tensor([11, 9], dtype=torch.int32)
    out = paged_decode_ref(q, kc, vc, ctx, bt, 0.5)
    perm = torch.tensor([7, 3, 0, 5, 1, 6, 2, 4])  # new block i holds old block perm[i]
    inv = torch.argsort(perm)
    out2 = paged_decode_ref(q, kc[perm], vc[perm], ctx, inv[bt.long()].to(torch.int32), 0.5)
    assert torch.allclose(out, out2, atol=1e-6)


def test_decode_gqa_equals_repeated_mha():
    kc, vc = _pool(4, 8, 2, 8, 7)
    q = torch.randn(2, 6, 8)
    bt = torch.tensor([[0, 1], [2, 3]], dtype=torch.int32)
    ctx = torch.tensor([13, 16], dtype=torch.int32)
    gqa = paged_decode_ref(q, kc, vc, ctx, bt, 0.4)
    mha = paged_decode_ref(q, kc.repeat_interleave(3, dim=2), vc.repeat_interleave(3, dim=2),
                           ctx, bt, 0.4)
    assert torch.allclose(gqa, mha, atol=1e-6)


# ---------------------------------------------------------------- prefill
def test_prefill_equal_lengths_is_sdpa_causal():
    g = torch.Generator().manual_seed(8)
    L = [5, 9]
    q = torch.randn(14, 4, 16, generator=g)
    k = torch.randn(14, 2, 16, generator=g)
    v = torch.randn(14, 2, 16, generator=g)
    cu = torch.tensor([0, 5, 14], dtype=torch.int32)
    ref = varlen_prefill_ref(q, k, v, cu, cu, 0.25)
    for i, (a, b) in enumerate([(0, 5), (5, 14)]):
        o = F.scaled_dot_product_attention(
            q[a:b].permute(1, 0, 2), k[a:b].permute(1, 0, 2).repeat_interleave(2, 0),
            v[a:b].permute(1, 0, 2).repeat_interleave(2, 0), is_causal=True, scale=0.25)
        assert torch.allclose(ref[a:b], o.permute(1, 0, 2), atol=1e-5)


def test_prefill_chunk_bottom_right_and_decode_row():
    kc, vc = _pool(6, 8, 2, 16, 9)
    g = torch.Generator().manual_seed(10)
    Lk, Lq = 21, 6
    bt = torch.tensor([[4, 0, 5]], dtype=torch.int32)
    q = torch.randn(Lk, 4, 16, generator=g)
    full = varlen_prefill_ref(q, kc, vc, torch.tensor([0, Lk], dtype=torch.int32),
                              torch.tensor([0, Lk], dtype=torch.int32), 0.3, block_tables=bt)
    chunk = varlen_prefill_ref(q[Lk - Lq:], kc, vc, torch.tensor([0, Lq], dtype=torch.int32),
                               torch.tensor([0, Lk], dtype=torch.int32), 0.3, block_tables=bt)
    assert torch.allclose(chunk, full[Lk - Lq:], atol=1e-5)  # chunked == one-shot rows
    dec = paged_decode_ref(q[Lk - 1:], kc, vc, torch.tensor([Lk], dtype=torch.int32), bt, 0.3)
    assert torch.allclose(full[-1], dec[0], atol=1e-5)  # last row == decode
    # first chunk row sees exactly Lk-Lq+1 keys
    dec2 = paged_decode_ref(q[Lk - Lq:Lk - Lq + 1], kc, vc,
                            torch.tensor([Lk - Lq + 1], dtype=torch.int32), bt, 0.3)
    assert torch.allclose(chunk[0], dec2[0], atol=1e-5)


def test_prefill_rows_equal_full_rows_and_decode():
    """varlen_prefill_rows_ref: the sampled rows of varlen_prefill_ref (chunked, GQA, paged),
    and each row equals decode over the keys it sees (Lk - Lq + pos + 1)."""
    kc, vc = _pool(12, 8, 2, 16, 21)
    g = torch.Generator().manual_seed(22)
    Lq, Lk = [5, 9, 1], [11, 9, 30]
    bt = torch.tensor([[3, 7, -1, -1], [0, 11, -1, -1], [9, 2, 5, 1]], dtype=torch.int32)
    cq = torch.tensor([0, 5, 14, 15], dtype=torch.int32)
    ck = torch.tensor([0, 11, 20, 50], dtype=torch.int32)
    q = torch.randn(15, 4, 16, generator=g)
    full = varlen_prefill_ref(q, kc, vc, cq, ck, 0.3, block_tables=bt)
    picks = [(0, 0), (0, 4), (1, 8), (1, 2), (2, 0), (0, 2)]
    seq = [s for s, _ in picks]
    pos = [p for _, p in picks]
    rows = torch.tensor([int(cq[s]) + p for s, p in picks])
    got = varlen_prefill_rows_ref(q[rows], seq, pos, kc, vc, cq, ck, 0.3, bt)
    assert torch.allclose(got, full[rows], atol=1e-6)
    for r, (s, p) in enumerate(picks):
        n = Lk[s] - Lq[s] + p + 1
        dec = paged_decode_ref(q[rows[r]:rows[r] + 1], kc, vc, torch.tensor([n], dtype=torch.int32),
                               bt[s:s + 1], 0.3)
        assert torch.allclose(got[r], dec[0], atol=1e-5)
