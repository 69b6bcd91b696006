"""ORACLE (test infrastructure): store_kvcache, paged decode, varlen prefill on CPU.

Follows nanokvllm/layers/attention.py:10-40 (store) and the semantics of the
flash-attn calls at attention.py:96-107 (decode: flash_attn_with_kvcache with
cache_seqlens and block_table; prefill: flash_attn_varlen_func, causal
bottom-right aligned when Lq < Lk). All attention math is fp32.
"""
from __future__ import annotations

import torch


def store_kvcache_ref(key, value, k_cache, v_cache, slot_mapping):
    """attention.py:21-30 + :33-40: row slot[i] of the flattened cache <- key[i]; -1 skipped.

    Mutates k_cache / v_cache (CPU tensors) in place.
    """
    N, Hk, D = key.shape
    kf = k_cache.view(-1, Hk * D)
    vf = v_cache.view(-1, Hk * D)
    slots = slot_mapping.to(torch.int64)
    keep = slots != -1
    idx = slots[keep]
    kf.index_copy_(0, idx, key.reshape(N, Hk * D)[keep])
    vf.index_copy_(0, idx, value.reshape(N, Hk * D)[keep])


def gather_paged_rows(cache, block_table_row, n_tokens):
    """Rows 0..n_tokens-1 of one sequence: cache[bt[t // B], t % B] -> [n, Hk, D]."""
    NB, B, Hk, D = cache.shape
    t = torch.arange(n_tokens)
    blocks = block_table_row.to(torch.int64)[t // B]
    return cache[blocks, t % B]


def paged_decode_ref(q, k_cache, v_cache, context_lens, block_tables, scale):
    """out[b, h] = softmax(scale * q[b,h] K_b^T) V_b over ctx_b keys, GQA h -> h // g.

    q [bs, Hq, D]; caches [NB, B, Hk, D]; returns fp32 [bs, Hq, D]
    (zeros for ctx <= 0).
    """
    bs, Hq, D = q.shape
    Hk = k_cache.size(2)
    g = Hq // Hk
    out = torch.zeros(bs, Hq, D, dtype=torch.float32)
    for b in range(bs):
        n = int(context_lens[b])
        if n <= 0:
            continue
        K = gather_paged_rows(k_cache, block_tables[b], n).float()  # [n, Hk, D]
        V = gather_paged_rows(v_cache, block_tables[b], n).float()
        Kh = K.permute(1, 0, 2).repeat_interleave(g, dim=0)  # [Hq, n, D]
        Vh = V.permute(1, 0, 2).repeat_interleave(g, dim=0)
        s = torch.bmm(q[b].float().unsqueeze(1), Kh.transpose(1, 2)).squeeze(1) * scale
        p = torch.softmax(s, dim=-1)
        out[b] = torch.bmm(p.unsqueeze(1), Vh).squeeze(1)
    return out


def varlen_prefill_ref(q, k, v, cu_seqlens_q, cu_seqlens_k, scale, block_tables=None):
    """Causal varlen attention; query j of a sequence sees keys 0 .. Lk-Lq+j.

    q [sum Lq, Hq, D]. With block_tables, k/v are paged caches [NB, B, Hk, D];
    otherwise contiguous [sum Lk, Hk, D]. Returns fp32 [sum Lq, Hq, D].
    """
    N, Hq, D = q.shape
    Hk = k.size(-2)
    g = Hq // Hk
    out = torch.zeros(N, Hq, D, dtype=torch.float32)
    n_seqs = cu_seqlens_q.numel() - 1
    for i in range(n_seqs):
        q0, q1 = int(cu_seqlens_q[i]), int(cu_seqlens_q[i + 1])
        k0, k1 = int(cu_seqlens_k[i]), int(cu_seqlens_k[i + 1])
        Lq, Lk = q1 - q0, k1 - k0
        if Lq == 0:
            continue
        if block_tables is not None:
            K = gather_paged_rows(k, block_tables[i], Lk).float()
            V = gather_paged_rows(v, block_tables[i], Lk).float()
        else:
            K, V = k[k0:k1].float(), v[k0:k1].float()
        Kh = K.permute(1, 0, 2).repeat_interleave(g, dim=0)  # [Hq, Lk, D]
        Vh = V.permute(1, 0, 2).repeat_interleave(g, dim=0)
        Q = q[q0:q1].float().permute(1, 0, 2)  # [Hq, Lq, D]
        s = torch.bmm(Q, Kh.transpose(1, 2)) * scale  # [Hq, Lq, Lk]
        jq = torch.arange(Lq).unsqueeze(1)
        tk = torch.arange(Lk).unsqueeze(0)
        s = s.masked_fill(tk > (Lk - Lq) + jq, float("-inf"))
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)  # fully masked rows (Lk < Lq) -> 0
        out[q0:q1] = torch.bmm(p, Vh).permute(1, 0, 2)
    return out


def varlen_prefill_rows_ref(q_rows, seq_of_row, pos_of_row, k_cache, v_cache, cu_seqlens_q,
                            cu_seqlens_k, scale, block_tables):
    """Selected output rows of varlen_prefill_ref (paged K/V), without the other rows.

    Row r is query pos_of_row[r] (0-based within its chunk) of sequence seq_of_row[r]:
    it sees keys 0 .. Lk-Lq+pos of that sequence (attention.py:96-102, bottom-right
    causal). q_rows [R, Hq, D]; returns fp32 [R, Hq, D]. The K/V of each sequence are
    gathered once for all of its rows, so long sequences cost O(rows * Lk).
    """
    R, Hq, D = q_rows.shape
    Hk = k_cache.size(-2)
    g = Hq // Hk
    out = torch.zeros(R, Hq, D, dtype=torch.float32)
    seq_of_row = torch.as_tensor(seq_of_row, dtype=torch.int64)
    pos_of_row = torch.as_tensor(pos_of_row, dtype=torch.int64)
    for i in sorted(set(seq_of_row.tolist())):
        rows = (seq_of_row == i).nonzero().view(-1)
        Lq = int(cu_seqlens_q[i + 1]) - int(cu_seqlens_q[i])
        Lk = int(cu_seqlens_k[i + 1]) - int(cu_seqlens_k[i])
        K = gather_paged_rows(k_cache, block_tables[i], Lk).float()
        V = gather_paged_rows(v_cache, block_tables[i], Lk).float()
        Kh = K.permute(1, 0, 2).repeat_interleave(g, dim=0)  # [Hq, Lk, D]
        Vh = V.permute(1, 0, 2).repeat_interleave(g, dim=0)
        Q = q_rows[rows].float().permute(1, 0, 2)  # [Hq, r, D]
        s = torch.bmm(Q, Kh.transpose(1, 2)) * scale  # [Hq, r, Lk]
        last = (Lk - Lq) + pos_of_row[rows].view(-1, 1)  # last visible key of each row
        s = s.masked_fill(torch.arange(Lk).view(1, -1) > last, float("-inf"))
        p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
        out[rows] = torch.bmm(p, Vh).permute(1, 0, 2)
    return out
