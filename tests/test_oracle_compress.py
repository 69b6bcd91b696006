"""Pins the oracle's compression step against brute force and closed forms (CPU).

Inputs plant the mistakes a restatement could make: a sink token with the
largest raw score (dropped -inf mask), heads that disagree (wrong head sum),
heads with different score spreads (dropped scale), the last window token
with a huge score (scored instead of always kept), and a per-slot brute force
of the two-phase compaction on tiny blocks.
"""
import math

import pytest
import torch

from oracle.compress_ref import (compress_compact_ref, get_tail_window_and_tail_slots_ref,
                                 select_topk_ref, snapkv_importance_ref, snapkv_ref)


def _brute_importance(Q, K, scale, agg):
    """float64 loops: softmax over keys 1..L-2 (key 0 masked, key L-1 unscored)."""
    m, Hk, L, D = K.shape
    Hq = Q.size(1)
    g = Hq // Hk
    n_sets = 1 if agg == "all" else Hk
    imp = torch.zeros(m, n_sets, L - 1, dtype=torch.float64)
    for b in range(m):
        for h in range(Hq):
            s = [float((Q[b, h, 0].double() * K[b, h // g, t].double()).sum()) * scale
                 for t in range(L - 1)]
            mx = max(s[1:])
            w = [0.0] + [math.exp(x - mx) for x in s[1:]]
            z = sum(w)
            for t in range(L - 1):
                imp[b, 0 if agg == "all" else h // g, t] += w[t] / z
    return imp


def _brute_topk(imp_row, k):
    idx = sorted(range(len(imp_row)), key=lambda i: (-float(imp_row[i]), i))[:k]
    return sorted(idx)


def _planted(seed, m=2, Hq=4, Hk=2, L=12, D=8):
    g = torch.Generator().manual_seed(seed)
    Q = torch.randn(m, Hq, 1, D, generator=g)
    K = torch.randn(m, Hk, L, D, generator=g)
    # sink: key 0 aligned with every query -> largest raw score
    K[:, :, 0] = Q[:, ::Hq // Hk, 0] * 4
    # last window token: huge score, must not influence the softmax
    K[:, :, L - 1] = Q[:, ::Hq // Hk, 0] * 8
    # head 1 of KV group 0 gets a 3x sharper spread (scale matters)
    Q[:, 1] *= 3
    return Q, K


@pytest.mark.parametrize("agg", ["all", "group"])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_importance_fp32_matches_brute_force(agg, seed):
    Q, K = _planted(seed)
    imp = snapkv_importance_ref(Q, K, 1, "fp32", agg)
    exp = _brute_importance(Q, K, K.size(-1) ** -0.5, agg)
    assert torch.allclose(imp.double(), exp, atol=1e-6)
    assert torch.all(imp[..., 0] == 0)  # sink masked


@pytest.mark.parametrize("agg", ["all", "group"])
def test_snapkv_fp32_matches_brute_force(agg):
    Q, K = _planted(3, m=3, L=16)
    num_keep = 5
    final = snapkv_ref(Q, K, None, num_keep=num_keep, window=1, score_dtype="fp32", agg=agg)
    exp_imp = _brute_importance(Q, K, K.size(-1) ** -0.5, agg)
    final = final.view(3, -1, num_keep + 2)
    for b in range(3):
        for s in range(final.size(1)):
            row = final[b, s].tolist()
            assert row[0] == 0 and row[-1] == 15 and len(row) == num_keep + 2
            assert row[1:-1] == _brute_topk(exp_imp[b, s].tolist(), num_keep)
            assert row[1:-1] == sorted(row[1:-1])


def test_snapkv_skip_rule():
    Q, K = _planted(4, L=8)
    assert snapkv_ref(Q, K, None, num_keep=7, window=1) is False  # L <= num_keep + window
    assert snapkv_ref(Q, K, None, num_keep=6, window=1) is not False


def test_topk_tie_rule_lower_index():
    imp = torch.tensor([[0.0, 0.5, 0.2, 0.5, 0.5, 0.1, 0.2]])
    assert select_topk_ref(imp, 2).tolist() == [[1, 3]]
    assert select_topk_ref(imp, 4).tolist() == [[1, 2, 3, 4]]
    assert select_topk_ref(imp, 5).tolist() == [[1, 2, 3, 4, 6]]


def test_bf16_path_equals_fp32_on_separated_scores():
    # keys of distinct, well separated strengths: bf16 rounding cannot reorder
    m, Hq, Hk, L, D = 2, 4, 2, 32, 16
    g = torch.Generator().manual_seed(5)
    Q = torch.zeros(m, Hq, 1, D)
    Q[:, :, 0, 0] = 1.0
    K = torch.zeros(m, Hk, L, D)
    strengths = torch.randperm(L, generator=g).float() * 0.5
    K[:, :, :, 0] = strengths * (D ** 0.5) / 4
    f32 = snapkv_ref(Q, K, None, num_keep=9, window=1, score_dtype="fp32")
    b16 = snapkv_ref(Q, K, None, num_keep=9, window=1, score_dtype="bf16")
    assert torch.equal(f32, b16)


# --------------------------------------------------------------- compaction
def _brute_compact(kc, vc, bt, lens, seq_idxs, B, W, keep_idx, keep_tokens):
    """Per-slot loop: snapshot the sources, then write the destinations."""
    kf, vf = kc.view(-1, kc.size(2), kc.size(3)), vc.view(-1, vc.size(2), vc.size(3))
    snap_k, snap_v = kf.clone(), vf.clone()
    for j, s in enumerate(seq_idxs):
        n = int(lens[s])
        full, tail = n // B, n % B
        wslot = [int(bt[s, full - W + p // B]) * B + p % B for p in range(W * B)]
        for i in range(keep_tokens):
            src = wslot[int(keep_idx[j, i])]
            kf[wslot[i]] = snap_k[src]
            vf[wslot[i]] = snap_v[src]
        for u in range(tail):
            src = int(bt[s, full]) * B + u
            dst = wslot[keep_tokens - 1] + 1 + u
            kf[dst] = snap_k[src]
            vf[dst] = snap_v[src]


@pytest.mark.parametrize("seed", [0, 1])
def test_compaction_matches_brute_force(seed):
    B, W, keep_blocks, extra = 4, 4, 2, 1
    keep_tokens = keep_blocks * B + extra  # 9 of a 16-token window
    g = torch.Generator().manual_seed(seed)
    nb, Hk, D = 24, 2, 4
    kc = torch.randn(nb, B, Hk, D, generator=g)
    vc = torch.randn(nb, B, Hk, D, generator=g)
    lens = torch.tensor([19, 16, 22, 9], dtype=torch.int32)  # tails 3, 0, 2, (too short)
    perm = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((4, 6), -1, dtype=torch.int32)
    p = 0
    for i, n in enumerate(lens.tolist()):
        nblk = math.ceil(n / B)
        bt[i, :nblk] = torch.tensor(perm[p:p + nblk])
        p += nblk
    seq_idxs = [0, 1, 2]
    q = torch.randn(4, 4, D, generator=g)
    kc2, vc2 = kc.clone(), vc.clone()
    ctx = lens.clone()
    ok, keep_idx, events = compress_compact_ref(
        q, kc2, vc2, bt, lens, ctx, seq_idxs, B, W, keep_blocks, extra, 0, 1,
        score_dtype="fp32")
    assert ok
    exp_k, exp_v = kc.clone(), vc.clone()
    _brute_compact(exp_k, exp_v, bt, lens, seq_idxs, B, W, keep_idx[:, 0], keep_tokens)
    assert torch.equal(kc2, exp_k) and torch.equal(vc2, exp_v)
    # closed forms: new_len = len - W*B + keep; keep_blocks = ceil(new_len / B)
    assert ctx.tolist() == [19 - 16 + 9, 16 - 16 + 9, 22 - 16 + 9, 9]
    for ev, s in zip(events, seq_idxs):
        n = int(lens[s])
        new_len = n - W * B + keep_tokens
        kb = math.ceil(new_len / B)
        assert ev["batch_index"] == s and ev["new_context_len"] == new_len
        assert ev["keep_blocks"] == kb
        nblk = math.ceil(n / B)
        assert ev["freed_block_ids"] == bt[s, kb:nblk].tolist()
        # full=F, tail=t: frees 1 block if t == 0 else 2 (W=4, keep=2B+1)
        assert len(ev["freed_block_ids"]) == (1 if n % B == 0 else 2)


def test_compaction_group_mode_moves_heads_independently():
    B, W = 4, 4
    g = torch.Generator().manual_seed(7)
    kc = torch.randn(8, B, 2, 4, generator=g)
    vc = torch.randn(8, B, 2, 4, generator=g)
    bt = torch.tensor([[0, 1, 2, 3, 4]], dtype=torch.int32)
    lens = torch.tensor([18], dtype=torch.int32)
    keep = torch.stack([torch.tensor([0, 2, 3, 5, 7, 8, 9, 12, 14, 15]),
                        torch.tensor([0, 1, 4, 6, 10, 11, 12, 13, 14, 15])]).unsqueeze(0)
    kc2, vc2 = kc.clone(), vc.clone()
    compress_compact_ref(None, kc2, vc2, bt, lens, lens.clone(), [0], B, W, 2, 2, 0, 2,
                         keep_idx=keep)
    kf, kf2 = kc.view(-1, 2, 4), kc2.view(-1, 2, 4)
    for h in range(2):
        for i in range(10):
            assert torch.equal(kf2[i, h], kf[int(keep[0, h, i]), h])
        for u in range(2):  # tail rows of block 4 follow the kept rows
            assert torch.equal(kf2[10 + u, h], kf[16 + u, h])


def test_window_location_closed_form():
    bt = torch.tensor([[7, 3, 9, 1, 4, 2], [5, 6, 8, 0, -1, -1]], dtype=torch.int32)
    lens = torch.tensor([21, 16], dtype=torch.int32)
    slots, old, tail, tail_ids = get_tail_window_and_tail_slots_ref(
        bt, lens, torch.tensor([0, 1]), 4, 3)
    assert slots[0].tolist() == [b * 4 + o for b in (9, 1, 4) for o in range(4)]
    assert slots[1].tolist() == [b * 4 + o for b in (6, 8, 0) for o in range(4)]
    assert tail.tolist() == [1, 0] and tail_ids.tolist() == [2, -1]


def _tiny_state(seed, B, lens, nb, Hk=2, D=4):
    g = torch.Generator().manual_seed(seed)
    kc = torch.randn(nb, B, Hk, D, generator=g)
    vc = torch.randn(nb, B, Hk, D, generator=g)
    perm = torch.randperm(nb, generator=g).tolist()
    width = max(math.ceil(n / B) for n in lens) + 1
    bt = torch.full((len(lens), width), -1, dtype=torch.int32)
    p = 0
    for i, n in enumerate(lens):
        k = math.ceil(n / B)
        bt[i, :k] = torch.tensor(perm[p:p + k])
        p += k
    return kc, vc, bt, torch.tensor(lens, dtype=torch.int32)


def _random_keep(g, m, n_sets, W, B, keep_tokens):
    """[0, ascending random middle, W*B - 1] per (sequence, set)."""
    rows = []
    for _ in range(m * n_sets):
        mid = torch.randperm(W * B - 2, generator=g)[:keep_tokens - 2] + 1
        rows.append(torch.cat([torch.tensor([0]), mid.sort().values, torch.tensor([W * B - 1])]))
    return torch.stack(rows).view(m, n_sets, keep_tokens)


@pytest.mark.parametrize("keep_blocks,extra", [(1, 1), (2, 1), (2, 2), (3, 0), (1, 3)])
def test_compaction_tail_where_the_reference_stays_in_block(keep_blocks, extra):
    """Tails that fit after the last kept token in its block ((keep-1) % B + tail < B): the
    oracle's logical placement equals the reference's slot(keep-1) + 1 + u, per slot."""
    B, W = 4, 4
    keep_tokens = keep_blocks * B + extra
    room = B - 1 - (keep_tokens - 1) % B  # tail rows that stay in the block
    lens = [W * B + t for t in range(0, room + 1)] + [(W + 1) * B + room]
    kc, vc, bt, lt = _tiny_state(11 + keep_tokens, B, lens, 40)
    sel = list(range(len(lens)))
    keep = _random_keep(torch.Generator().manual_seed(keep_tokens), len(sel), 1, W, B,
                        keep_tokens)
    kc2, vc2 = kc.clone(), vc.clone()
    compress_compact_ref(None, kc2, vc2, bt, lt, lt.clone(), sel, B, W, keep_blocks, extra, 0,
                         1, keep_idx=keep)
    exp_k, exp_v = kc.clone(), vc.clone()
    _brute_compact(exp_k, exp_v, bt, lt, sel, B, W, keep[:, 0], keep_tokens)
    assert torch.equal(kc2, exp_k) and torch.equal(vc2, exp_v)


def _read_seq(cache, bt_row, n, B):
    return torch.stack([cache[int(bt_row[t // B]), t % B] for t in range(n)])


@pytest.mark.parametrize("agg_sets", [1, 2])
@pytest.mark.parametrize("keep_blocks,extra", [(2, 0), (1, 3), (2, 2), (3, 0)])
def test_compaction_read_back_through_the_table(agg_sets, keep_blocks, extra):
    """Any keep and tail: the compacted sequence read through its block table is its
    prefix, then the kept window rows in order, then the tail rows; every slot outside the
    sequence's own blocks is untouched. (Where keep % B + tail > B the reference's
    slot(keep-1) + 1 + u lies past the last kept token's block.)"""
    B, W = 4, 4
    keep_tokens = keep_blocks * B + extra
    lens = [W * B + 3, W * B + 1, (W + 2) * B + 2, W * B, (W + 1) * B + 3]
    kc, vc, bt, lt = _tiny_state(5 + keep_tokens * agg_sets, B, lens, 48)
    sel = [0, 1, 2, 3, 4]
    keep = _random_keep(torch.Generator().manual_seed(3 + keep_tokens), len(sel), agg_sets, W,
                        B, keep_tokens)
    kc2, vc2, ctx = kc.clone(), vc.clone(), lt.clone()
    compress_compact_ref(None, kc2, vc2, bt, lt, ctx, sel, B, W, keep_blocks, extra, 0, 1,
                         keep_idx=keep)
    owned = {int(b) for b in bt.flatten().tolist() if b >= 0}
    for b in range(kc.size(0)):
        if b not in owned:
            assert torch.equal(kc2[b], kc[b]) and torch.equal(vc2[b], vc[b])
    for j, s in enumerate(sel):
        n, new_n = lens[s], int(ctx[s])
        assert new_n == n - W * B + keep_tokens
        w0 = (n // B - W) * B
        for old_c, new_c in ((kc, kc2), (vc, vc2)):
            old = _read_seq(old_c, bt[s], n, B)
            new = _read_seq(new_c, bt[s], new_n, B)
            assert torch.equal(new[:w0], old[:w0])
            for h in range(kc.size(2)):
                ki = keep[j, 0 if agg_sets == 1 else h]
                assert torch.equal(new[w0:w0 + keep_tokens, h], old[w0 + ki, h])
            assert torch.equal(new[w0 + keep_tokens:], old[w0 + W * B:])


def test_compaction_read_back_fails_for_the_physical_rule():
    """A planted mistake: placing the tail at slot(keep-1) + 1 + u (the reference's rule)
    where it leaves the block breaks the read-back of the previous test."""
    B, W, keep_tokens = 4, 4, 8  # keep_blocks 2, extra 0: every tail leaves the block
    lens = [W * B + 3]
    kc, vc, bt, lt = _tiny_state(1, B, lens, 12)
    keep = _random_keep(torch.Generator().manual_seed(1), 1, 1, W, B, keep_tokens)
    exp_k, exp_v = kc.clone(), vc.clone()
    _brute_compact(exp_k, exp_v, bt, lt, [0], B, W, keep[:, 0], keep_tokens)
    new_n = lens[0] - W * B + keep_tokens
    new = _read_seq(exp_k, bt[0], new_n, B)
    old = _read_seq(kc, bt[0], lens[0], B)
    assert not torch.equal(new[keep_tokens:], old[W * B:])


def test_gather_kv_by_slots_explicit_loops():
    """gather_kv_by_slots_ref (compress_utils.py:75-97): k_sub[j, h, p] = k_cache[s // B,
    s % B, h] for s = slots[j, p], by loops; a planted head/position transposition fails."""
    from oracle.compress_ref import gather_kv_by_slots_ref
    g = torch.Generator().manual_seed(8)
    NB, B, Hk, D = 6, 4, 3, 5
    kc = torch.randn(NB, B, Hk, D, generator=g)
    vc = torch.randn(NB, B, Hk, D, generator=g)
    slots = torch.stack([torch.randperm(NB * B, generator=g)[:7] for _ in range(2)])
    k_sub, v_sub = gather_kv_by_slots_ref(kc, vc, slots)
    assert k_sub.shape == (2, Hk, 7, D) and k_sub.is_contiguous()
    for j in range(2):
        for h in range(Hk):
            for p in range(7):
                s = int(slots[j, p])
                assert torch.equal(k_sub[j, h, p], kc[s // B, s % B, h])
                assert torch.equal(v_sub[j, h, p], vc[s // B, s % B, h])
    # the planted mistake: heads and positions swapped (no permute) reads other rows
    wrong = kc.view(NB * B, Hk, D)[slots]  # [2, 7, Hk, D]
    assert not torch.equal(wrong.reshape(2, Hk, 7, D), k_sub)


def _brute_importance_window(Q, K, scale, agg, w):
    """float64 loops with a query window of w tokens: each window query's softmax over
    keys 1 .. L-w-1 (key 0 masked, the window keys unscored), summed over queries and heads."""
    m, Hk, L, D = K.shape
    Hq = Q.size(1)
    g = Hq // Hk
    n = L - w
    imp = torch.zeros(m, 1 if agg == "all" else Hk, n, dtype=torch.float64)
    for b in range(m):
        for h in range(Hq):
            for i in range(w):
                s = [float((Q[b, h, i].double() * K[b, h // g, t].double()).sum()) * scale
                     for t in range(n)]
                mx = max(s[1:])
                e = [0.0] + [math.exp(x - mx) for x in s[1:]]
                z = sum(e)
                for t in range(n):
                    imp[b, 0 if agg == "all" else h // g, t] += e[t] / z
    return imp


@pytest.mark.parametrize("agg", ["all", "group"])
@pytest.mark.parametrize("w", [2, 3])
def test_importance_query_window_matches_brute_force(agg, w):
    """SnapKV's window (CompressMethod.py:14-42): the softmax of every window query is
    summed over the window, then over heads; the window keys are not candidates."""
    g = torch.Generator().manual_seed(40 + w)
    m, Hq, Hk, L, D = 2, 4, 2, 14, 8
    Q = torch.randn(m, Hq, w, D, generator=g)
    K = torch.randn(m, Hk, L, D, generator=g)
    Q[:, 1] *= 3  # a sharper head
    imp = snapkv_importance_ref(Q, K, w, "fp32", agg)
    exp = _brute_importance_window(Q, K, D ** -0.5, agg, w)
    assert imp.shape == exp.shape
    assert torch.allclose(imp.double(), exp, atol=1e-6)
    final = snapkv_ref(Q, K, None, num_keep=4, window=w, score_dtype="fp32", agg=agg)
    final = final.view(m, -1, 4 + 1 + w)
    for b in range(m):
        for s_ in range(final.size(1)):
            row = final[b, s_].tolist()
            assert row[0] == 0 and row[-w:] == list(range(L - w, L))
            assert row[1:5] == _brute_topk(exp[b, s_].tolist(), 4)
