"""ORACLE (test infrastructure): the window-based periodic compression step on CPU.

Restates nanokvllm/layers/compress_utils.py:9-290 and
nanokvllm/layers/CompressMethod.py:4-57 with torch CPU ops in the same order
and dtypes (score_dtype="bf16", the reference) or in fp32 (score_dtype="fp32",
what the HIP kernels compute). The reference's torch.topk(sorted=False) has no
documented tie order; the oracle fixes one: larger importance first, then the
lower index. agg="group" (one kept set per KV head, summing the g query heads
of that KV head) is the per-KV-head variant; agg="all" is the reference.
"""
from __future__ import annotations

import numpy as np
import torch


def get_tail_window_and_tail_slots_ref(block_tables, context_lens, seq_idxs, block_size,
                                       window_blocks):
    """compress_utils.py:9-72: window slots [m, W*B], lens, tail lens, tail block ids."""
    old = context_lens.index_select(0, seq_idxs).to(torch.long)
    bt = block_tables.index_select(0, seq_idxs).to(torch.long)
    B = block_size
    m = seq_idxs.numel()
    full = old // B
    tail = old % B
    assert torch.all(full >= window_blocks), f"some full_blocks < window_blocks: {full}"
    wb_idx = (full - window_blocks).unsqueeze(1) + torch.arange(window_blocks).view(1, -1)
    wb_ids = torch.gather(bt, 1, wb_idx)
    assert torch.all(wb_ids >= 0)
    slots = (wb_ids.unsqueeze(-1) * B + torch.arange(B).view(1, 1, B)).reshape(m, window_blocks * B)
    safe = torch.clamp(full, max=bt.size(1) - 1)
    tail_ids = torch.gather(bt, 1, safe.unsqueeze(1)).squeeze(1)
    tail_ids = torch.where(tail > 0, tail_ids, torch.full_like(tail_ids, -1))
    return slots, old, tail, tail_ids


def gather_kv_by_slots_ref(k_cache, v_cache, src_slots):
    """compress_utils.py:75-97: [m, S] slots -> K/V [m, Hk, S, D]."""
    NB, B, Hk, D = k_cache.shape
    kf = k_cache.view(NB * B, Hk, D)
    vf = v_cache.view(NB * B, Hk, D)
    return (kf[src_slots].permute(0, 2, 1, 3).contiguous(),
            vf[src_slots].permute(0, 2, 1, 3).contiguous())


def snapkv_importance_ref(Q, K, window=1, score_dtype="bf16", agg="all"):
    """CompressMethod.py:14-42: key importance [m, n_sets, L-window].

    bf16: matmul, scale, softmax and both sums in bf16 tensors as the
    reference; fp32: the same ops on fp32 copies.
    """
    m, Hk, L, D = K.shape
    Hq = Q.size(1)
    dt = torch.bfloat16 if score_dtype == "bf16" else torch.float32
    Qd, Kd = Q.to(dt), K.to(dt)
    K_cut = Kd[:, :, :-window, :]
    scale = 1.0 / (D ** 0.5)
    if Hq == Hk:
        s = torch.matmul(Qd, K_cut.transpose(-1, -2)) * scale
    else:
        g = Hq // Hk
        Qg = Qd.view(m, Hk, g, window, D)
        Kt = K_cut.transpose(-1, -2).unsqueeze(2).contiguous()
        s = (torch.matmul(Qg, Kt) * scale).view(m, Hq, window, L - window)
    s[:, :, :, 0] = -float("inf")
    p = torch.softmax(s, dim=-1)
    imp = p.sum(dim=2)  # [m, Hq, L-window]
    if agg == "all":
        if imp.size(1) > 1:
            imp = imp.sum(dim=1, keepdim=True)
    else:
        g = Hq // Hk
        imp = imp.view(m, Hk, g, L - window).sum(dim=2)
    return imp


def select_topk_ref(importance, num_keep):
    """Top num_keep per row (larger first, ties -> lower index), ascending.

    importance [..., n] (any float dtype) -> int64 [..., num_keep].
    """
    x = importance.detach().to(torch.float64).cpu().numpy()
    flat = x.reshape(-1, x.shape[-1])
    out = np.empty((flat.shape[0], num_keep), dtype=np.int64)
    for r in range(flat.shape[0]):
        order = np.argsort(-flat[r], kind="stable")  # stable: equal values keep index order
        out[r] = np.sort(order[:num_keep])
    return torch.from_numpy(out.reshape(*x.shape[:-1], num_keep))


def snapkv_ref(Q, K, V=None, num_keep=220, window=1, score_dtype="bf16", agg="all"):
    """CompressMethod.py:4-57 -> final_idx [m, (n_sets,) 1 + num_keep + window] or False."""
    m, Hk, L, D = K.shape
    if L - window <= 0 or L <= num_keep + window:
        return False
    imp = snapkv_importance_ref(Q, K, window, score_dtype, agg)  # [m, n_sets, L-window]
    keep = select_topk_ref(imp, num_keep)  # [m, n_sets, num_keep]
    n_sets = keep.size(1)
    bos = torch.zeros(m, n_sets, 1, dtype=torch.long)
    tail = torch.arange(L - window, L).view(1, 1, -1).expand(m, n_sets, window)
    final = torch.cat([bos, keep, tail], dim=-1)
    return final.view(m, -1) if agg == "all" else final


def compress_compact_ref(q_current, k_cache, v_cache, block_tables, base_context_lens,
                         context_lens, seq_idxs, block_size, window_blocks, keep_blocks,
                         keep_extra_tokens, layer_id, num_layers, score_dtype="bf16", agg="all",
                         keep_idx=None):
    """MyCompressCompact (compress_utils.py:100-290) on CPU tensors, in place.

    Returns (ok, keep_idx [m, n_sets, keep_tokens], events or None). If
    keep_idx is given, scoring is skipped and those positions are used.
    Tail row u goes to logical position keep_tokens + u of the window region
    (window blocks, then the tail block), which is the reference's slot
    wherever the reference stays inside the last kept block.
    """
    seq_idxs = torch.as_tensor(seq_idxs, dtype=torch.long)
    m = seq_idxs.numel()
    if m == 0:
        return False, None, None
    B = block_size
    window_tokens = window_blocks * B
    keep_tokens = keep_blocks * B + keep_extra_tokens
    slots, old, tail_lens, tail_ids = get_tail_window_and_tail_slots_ref(
        block_tables, base_context_lens, seq_idxs, B, window_blocks)
    NB, _, Hk, D = k_cache.shape
    if keep_idx is None:
        q_sub = q_current.index_select(0, seq_idxs).unsqueeze(2)
        k_sub, _ = gather_kv_by_slots_ref(k_cache, v_cache, slots)
        final = snapkv_ref(q_sub, k_sub, None, num_keep=keep_tokens - 2, window=1,
                           score_dtype=score_dtype, agg=agg)
        if final is False:
            return False, None, None
        keep_idx = final.view(m, 1, -1) if agg == "all" else final
    keep_idx = keep_idx.to(torch.long)
    n_sets = keep_idx.size(1)
    assert keep_idx.size(2) == keep_tokens
    assert int(keep_idx.min()) >= 0 and int(keep_idx.max()) < window_tokens

    new_lens = old - window_tokens + keep_tokens
    dst_keep = slots[:, :keep_tokens]  # [m, keep]
    # the window's slots followed by the tail block's: logical position p of the window
    # region (p < W*B + B) is slot ext[:, p]
    tail_slots = tail_ids.clamp(min=0).unsqueeze(1) * B + torch.arange(B).view(1, B)
    ext = torch.cat([slots, tail_slots], dim=1)
    total_slots = NB * B
    kf = k_cache.view(total_slots, Hk, D)
    vf = v_cache.view(total_slots, Hk, D)
    for s in range(n_sets):
        heads = slice(None) if n_sets == 1 else slice(s, s + 1)
        src_keep = torch.gather(slots, 1, keep_idx[:, s, :])
        src = [src_keep.reshape(-1)]
        dst = [dst_keep.reshape(-1)]
        for i in range(m):  # tail part (compress_utils.py:210-231)
            t = int(tail_lens[i])
            if t > 0:
                off = torch.arange(t)
                src.append(tail_ids[i] * B + off)
                # logical position keep_tokens + u; the reference's physical slot
                # dst_keep[-1] + 1 + u equals it while it stays inside the last kept
                # block (keep_tokens % B + tail <= B, e.g. the default 2*B + 1 keep)
                # and would land in an unrelated block past it
                dst.append(ext[i, keep_tokens + off])
        src_flat = torch.cat(src)
        dst_flat = torch.cat(dst)
        assert int(src_flat.min()) >= 0 and int(src_flat.max()) < total_slots
        assert int(dst_flat.min()) >= 0 and int(dst_flat.max()) < total_slots
        # two-phase stable compaction (compress_utils.py:256-260)
        vals_k = kf[:, heads].index_select(0, src_flat).clone()
        vals_v = vf[:, heads].index_select(0, src_flat).clone()
        kh = kf[:, heads]
        vh = vf[:, heads]
        kh.index_copy_(0, dst_flat, vals_k)
        vh.index_copy_(0, dst_flat, vals_v)
        if n_sets > 1:
            kf[:, heads] = kh
            vf[:, heads] = vh
    context_lens[seq_idxs] = new_lens.to(context_lens.dtype)

    events = None
    if layer_id + 1 >= num_layers:
        bt = block_tables.index_select(0, seq_idxs).to(torch.long)
        keep_after = (new_lens + B - 1) // B
        events = []
        for i, bidx in enumerate(seq_idxs.tolist()):
            kb = int(keep_after[i])
            freed = [int(x) for x in bt[i, kb:].tolist() if int(x) >= 0]
            events.append({
                "batch_index": int(bidx), "layer": int(layer_id),
                "new_context_len": int(new_lens[i]), "keep_blocks": kb,
                "freed_block_ids": freed, "tail_uncompressed_len_after": 0,
            })
    return True, keep_idx, events


def compress_schedule_ref(context_lens, tail_uncompressed, block_size, window_blocks, topk,
                          counter, period, policy="first"):
    """model_runner.py:300-332: counter += 1; on every period-th step sequence i is eligible
    iff len % B != B - 1, tail_uncompressed >= W*B and len // B >= W; the first topk
    eligible in batch order ("first", the reference) or the topk longest ("longest", ties
    to the lower index). Returns (new counter, selected indices, fired)."""
    counter += 1
    fired = counter % period == 0
    if not fired:
        return counter, [], False
    B = block_size
    cand = [i for i, (n, t) in enumerate(zip(context_lens, tail_uncompressed))
            if n % B != B - 1 and t >= window_blocks * B and n // B >= window_blocks]
    if policy == "longest":
        cand.sort(key=lambda i: (-context_lens[i], i))
    return counter, cand[:topk], True
