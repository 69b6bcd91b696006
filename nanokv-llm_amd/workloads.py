"""Seeded synthetic inputs for the paged-attention workloads (no checkpoints).

Each generator builds a paged K/V pool ``[n_blocks, 256, Hk, 128]`` (bf16; K and
V are the two halves of one ``[2, n_blocks, ...]`` tensor, as the reference's
pool holds them), assigns every sequence ``ceil(ctx / B)`` physical blocks drawn without
replacement from a random permutation of the pool, and derives block tables
(right-padded with -1) and the slot of the newest token. Integer choices use
a CPU ``torch.Generator`` seeded with ``seed`` so they are identical on every
machine; the bulk random values are drawn on ``device``.

Workloads (sizes from the reference's Qwen3 geometries, block size 256):
  decode_qwen3_0_6b   bs 4,  Hq 16, Hk 8, ctx U[300, 1000], pool 16 blocks,
                      q/K/V ~ N(0,1)/sqrt(128)
  decode_qwen3_8b     bs 64, Hq 32, Hk 8, ctx U[2048, 8192], pool 4096 blocks,
                      q/K/V ~ N(0,1); one new token per sequence stored first
  compress_qwen3_8b   bs 500, Hq 32, Hk 8, ctx U[1500, 4096], top-20 longest,
                      W = 4 blocks, keep 2*256+1
  prefill_qwen3_8b    16 sequences, L U[512, 4096]; chunked: 2048-token chunks
                      on paged prefixes of U[0, 8192] tokens
  decode_qwen3_32b_longctx  bs 500, Hq 64, Hk 8, ctx log-uniform [1024, 16384], 20%
                      of the sequences already compressed once (shorter context),
                      a pool sized to fill most of HBM with only the used blocks
                      written
  compress_qwen3_32b_longctx  the compression step on that state: the 20 longest
                      sequences eligible under the engine's rule, W = 4 blocks,
                      keep 2*256+1, only the selected sequences owning blocks
"""
from __future__ import annotations

import math

import torch

BLOCK = 256
HEAD_DIM = 128


def _randn(shape, gen_seed, device, dtype=torch.bfloat16, scale=1.0):
    g = torch.Generator(device=device)
    g.manual_seed(gen_seed)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if scale != 1.0:
        x.mul_(scale)
    return x.to(dtype)


def _kv_pool(shape, seed, device, scale=1.0):
    """K and V caches laid out as the reference allocates them: the two halves of one
    [2, num_blocks, block_size, Hk, D] tensor (nanokvllm/engine/model_runner.py:145, one
    layer), filled as _randn(shape, seed*7+1) and _randn(shape, seed*7+2) would be."""
    kv = torch.empty((2,) + tuple(shape), dtype=torch.bfloat16, device=device)
    kv[0].copy_(_randn(shape, seed * 7 + 1, device, scale=scale))
    kv[1].copy_(_randn(shape, seed * 7 + 2, device, scale=scale))
    return kv[0], kv[1]


def assign_blocks(ctx_lens: list[int], n_blocks: int, gen: torch.Generator, block=BLOCK,
                  extra_tokens: int = 0):
    """Block tables for sequences of the given lengths (+extra_tokens headroom)."""
    need = [math.ceil((c + extra_tokens) / block) for c in ctx_lens]
    total = sum(need)
    if total > n_blocks:
        raise ValueError(f"pool of {n_blocks} blocks cannot hold {total} blocks")
    perm = torch.randperm(n_blocks, generator=gen)[:total].tolist()
    width = max(need)
    tables, pos = [], 0
    for n in need:
        tables.append(perm[pos:pos + n] + [-1] * (width - n))
        pos += n
    return torch.tensor(tables, dtype=torch.int32)


def slot_of(block_tables: torch.Tensor, positions: torch.Tensor, block=BLOCK):
    """slot = block_table[b, pos // B] * B + pos % B (model_runner.py:192-194)."""
    pos = positions.to(torch.int64)
    blk = torch.gather(block_tables.to(torch.int64), 1, (pos // block).view(-1, 1)).view(-1)
    return (blk * block + pos % block).to(torch.int32)


def decode_workload(bs, Hq, Hk, ctx_lo, ctx_hi, n_blocks, seed, device="cpu", value_scale=1.0,
                    n_table_sets=1, head_dim=HEAD_DIM):
    """Paged decode inputs; context lengths include the token stored this step.

    Returns a dict with q [bs,Hq,D], new key/value [bs,Hk,D], k_cache/v_cache,
    context_lens [bs] (int32), slot_mapping [bs] and block_tables (a list of
    n_table_sets independent random assignments of the same lengths).
    """
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (bs,), generator=gen, dtype=torch.int64)
    tables = [assign_blocks(ctx.tolist(), n_blocks, gen) for _ in range(n_table_sets)]
    D = head_dim
    k_cache, v_cache = _kv_pool((n_blocks, BLOCK, Hk, D), seed, device, scale=value_scale)
    q = _randn((bs, Hq, D), seed * 7 + 3, "cpu", scale=value_scale)
    key = _randn((bs, Hk, D), seed * 7 + 4, "cpu", scale=value_scale)
    value = _randn((bs, Hk, D), seed * 7 + 5, "cpu", scale=value_scale)
    ctx32 = ctx.to(torch.int32)
    return dict(q=q, key=key, value=value, k_cache=k_cache, v_cache=v_cache,
                context_lens=ctx32, block_tables=tables,
                slot_mappings=[slot_of(t, ctx - 1) for t in tables],
                scale=D ** -0.5, Hq=Hq, Hk=Hk)


def decode_qwen3_0_6b(seed=1, device="cpu"):
    return decode_workload(4, 16, 8, 300, 1000, 16, seed, device, value_scale=HEAD_DIM ** -0.5)


def decode_qwen3_8b(seed=2, device="cpu", bs=64, n_blocks=4096, n_table_sets=1):
    return decode_workload(bs, 32, 8, 2048, 8192, n_blocks, seed, device,
                           n_table_sets=n_table_sets)


def compress_workload(bs, Hq, Hk, ctx_lo, ctx_hi, topk, seed, device="cpu", n_blocks=None,
                      selected_only=False, head_dim=HEAD_DIM):
    """Decode state for a compression step; selection = the topk longest sequences.

    With selected_only, only the selected sequences get blocks (the others
    keep their lengths but own no cache) -- enough for the step itself.
    """
    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(ctx_lo, ctx_hi + 1, (bs,), generator=gen, dtype=torch.int64)
    order = sorted(range(bs), key=lambda i: (-int(ctx[i]), i))
    selected = sorted(order[:topk])
    lens_for_tables = [int(ctx[i]) if (not selected_only or i in selected) else 0
                       for i in range(bs)]
    need = sum(math.ceil(c / BLOCK) for c in lens_for_tables)
    n_blocks = n_blocks or need + 8
    table = assign_blocks(lens_for_tables, n_blocks, gen)
    D = head_dim
    k_cache, v_cache = _kv_pool((n_blocks, BLOCK, Hk, D), seed, device)
    q = _randn((bs, Hq, D), seed * 7 + 3, "cpu")
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, context_lens=ctx.to(torch.int32),
                block_tables=table, seq_idx=selected, Hq=Hq, Hk=Hk)


def compress_qwen3_8b(seed=3, device="cpu", selected_only=True):
    return compress_workload(500, 32, 8, 1500, 4096, 20, seed, device,
                             selected_only=selected_only)


def prefill_workload(n_seqs, Hq, Hk, len_lo, len_hi, seed, device="cpu", prefix_lo=None,
                     prefix_hi=None, chunk=None, head_dim=HEAD_DIM, block_size=BLOCK):
    """Varlen prefill over the paged cache.

    One-shot: Lq = Lk = L ~ U[len_lo, len_hi]. Chunked (chunk given): prefix
    P ~ U[prefix_lo, prefix_hi] already in cache, Lq = chunk, Lk = P + chunk.
    The new chunk's K/V rows (key/value) are what store_kvcache writes before
    the attention; the cache holds N(0,1) values for the prefix.
    """
    gen = torch.Generator().manual_seed(seed)
    if chunk is None:
        Lq = torch.randint(len_lo, len_hi + 1, (n_seqs,), generator=gen).tolist()
        Lk = list(Lq)
    else:
        P = torch.randint(prefix_lo, prefix_hi + 1, (n_seqs,), generator=gen).tolist()
        Lq = [chunk] * n_seqs
        Lk = [p + chunk for p in P]
    B = block_size
    need = sum(math.ceil(k / B) for k in Lk)
    n_blocks = need + 8
    table = assign_blocks(Lk, n_blocks, gen, block=B)
    cu_q = torch.tensor([0] + list(torch.tensor(Lq).cumsum(0).tolist()), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(Lk).cumsum(0).tolist()), dtype=torch.int32)
    N = int(cu_q[-1])
    D = head_dim
    positions = torch.cat([torch.arange(k - q, k) for q, k in zip(Lq, Lk)])
    seq_of = torch.cat([torch.full((q,), i, dtype=torch.int64) for i, q in enumerate(Lq)])
    blk = table.to(torch.int64)[seq_of, positions // B]
    slots = (blk * B + positions % B).to(torch.int32)
    k_cache, v_cache = _kv_pool((n_blocks, B, Hk, D), seed, device)
    return dict(
        q=_randn((N, Hq, D), seed * 7 + 3, device),
        key=_randn((N, Hk, D), seed * 7 + 4, device),
        value=_randn((N, Hk, D), seed * 7 + 5, device),
        k_cache=k_cache, v_cache=v_cache,
        block_tables=table, cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, slot_mapping=slots,
        max_seqlen_q=max(Lq), max_seqlen_k=max(Lk), Lq=Lq, Lk=Lk, Hq=Hq, Hk=Hk,
        scale=D ** -0.5, positions=positions.to(device))


def prefill_qwen3_8b(seed=4, device="cpu", n_seqs=16):
    return prefill_workload(n_seqs, 32, 8, 512, 4096, seed, device)


def prefill_chunked_qwen3_8b(seed=5, device="cpu", n_seqs=16):
    return prefill_workload(n_seqs, 32, 8, 0, 0, seed, device, prefix_lo=0, prefix_hi=8192,
                            chunk=2048)


def decode_bytes(context_lens, Hq, Hk, D=HEAD_DIM, max_blocks=0):
    """Algorithmic HBM bytes of one paged decode call (K+V rows, q, out, tables)."""
    ctx = int(torch.as_tensor(context_lens).to(torch.int64).clamp(min=0).sum())
    bs = int(torch.as_tensor(context_lens).numel())
    return ctx * Hk * D * 2 * 2 + bs * Hq * D * 2 * 2 + bs * 4 * (max_blocks + 1)


def decode_qwen3_32b_longctx(seed=6, device="cpu", bs=500, n_blocks=None, frac_compressed=0.2,
                             pool_fraction=0.85, window_tokens=1024, keep_tokens=513,
                             alloc_caches=True):
    """High-concurrency long-context decode state at Qwen3-32B geometry.

    Context lengths exp(U(ln 1024, ln 16384)); a random 20% of the sequences were
    compressed once before (len - window_tokens + keep_tokens: their kept middle
    positions are non-contiguous, which for attention is just a shorter context)
    and have no uncompressed tail yet. The pool defaults to pool_fraction of the
    device's free memory for K+V (at most 0.85 * 288 GB / 1 MiB blocks); blocks
    are assigned at random over the whole pool and only the used ones are filled
    with N(0,1) values. Returns decode_workload's fields plus ``compressed``
    (bool per sequence) and ``tail_uncompressed`` (tokens since the last
    compression).
    With alloc_caches=False the caches are None (tables and lengths only).
    """
    gen = torch.Generator().manual_seed(seed)
    u = torch.rand(bs, generator=gen, dtype=torch.float64)
    ctx = torch.exp(math.log(1024) + u * (math.log(16384) - math.log(1024))).to(torch.int64)
    compressed = torch.rand(bs, generator=gen) < frac_compressed
    ctx = torch.where(compressed, ctx - window_tokens + keep_tokens, ctx)
    tail_unc = torch.where(compressed, torch.zeros_like(ctx), ctx)
    Hq, Hk, D = 64, 8, HEAD_DIM
    block_bytes = 2 * BLOCK * Hk * D * 2
    if n_blocks is None:
        if torch.device(device).type == "cuda":
            free, _ = torch.cuda.mem_get_info(torch.device(device))
            n_blocks = int(free * pool_fraction) // block_bytes
        else:
            n_blocks = 0
        n_blocks = min(max(n_blocks, 0), int(0.85 * 288e9) // (1 << 20))
    need = sum(math.ceil(int(c) / BLOCK) for c in ctx.tolist())
    n_blocks = max(n_blocks, need + 8)
    table = assign_blocks(ctx.tolist(), n_blocks, gen)
    k_cache = v_cache = None
    used = table[table >= 0].to(torch.int64)
    if alloc_caches:  # one [2, n_blocks, ...] tensor, as the reference's pool
        kv = torch.empty(2, n_blocks, BLOCK, Hk, D, dtype=torch.bfloat16, device=device)
        k_cache, v_cache = kv[0], kv[1]
        g = torch.Generator(device=device)
        g.manual_seed(seed * 7 + 1)
    for i in range(0, used.numel() if alloc_caches else 0, 1024):  # used blocks, 1 GiB a time
        ids = used[i:i + 1024].to(device)
        k_cache[ids] = torch.randn((ids.numel(), BLOCK, Hk, D), generator=g, device=device,
                                   dtype=torch.float32).to(torch.bfloat16)
        v_cache[ids] = torch.randn((ids.numel(), BLOCK, Hk, D), generator=g, device=device,
                                   dtype=torch.float32).to(torch.bfloat16)
    q = _randn((bs, Hq, D), seed * 7 + 3, "cpu")
    key = _randn((bs, Hk, D), seed * 7 + 4, "cpu")
    value = _randn((bs, Hk, D), seed * 7 + 5, "cpu")
    return dict(q=q, key=key, value=value, k_cache=k_cache, v_cache=v_cache,
                context_lens=ctx.to(torch.int32), block_tables=[table],
                slot_mappings=[slot_of(table, ctx - 1)], scale=D ** -0.5, Hq=Hq, Hk=Hk,
                compressed=compressed, tail_uncompressed=tail_unc, n_blocks=n_blocks)


def eligible_longest(context_lens, tail_uncompressed, topk, block=BLOCK, window_blocks=4):
    """The topk longest sequences (ties to the lower index) that the engine's scheduling rule
    admits to a compression step (nanokvllm/engine/model_runner.py:313-323): len % B != B-1,
    tokens since the last compression >= W*B and len // B >= W. Returned in batch order."""
    lens = [int(x) for x in context_lens]
    tails = [int(x) for x in tail_uncompressed]
    elig = [i for i, n in enumerate(lens)
            if n % block != block - 1 and tails[i] >= window_blocks * block
            and n // block >= window_blocks]
    return sorted(sorted(elig, key=lambda i: (-lens[i], i))[:topk])


def compress_qwen3_32b_longctx(seed=6, device="cpu", topk=20):
    """The compression step of the long-context decode state at Qwen3-32B geometry (Hq 64,
    Hk 8, batch 500): the lengths, tails and q of decode_qwen3_32b_longctx(seed), the topk
    longest eligible sequences selected, and a compact pool in which only those sequences own
    blocks (whole tables, up to 64 blocks each; the others keep their lengths and no cache)."""
    st = decode_qwen3_32b_longctx(seed=seed, alloc_caches=False)
    lens = st["context_lens"]
    sel = eligible_longest(lens.tolist(), st["tail_uncompressed"].tolist(), topk)
    gen = torch.Generator().manual_seed(seed * 7 + 6)
    lens_for_tables = [int(lens[i]) if i in sel else 0 for i in range(lens.numel())]
    n_blocks = sum(math.ceil(c / BLOCK) for c in lens_for_tables) + 8
    table = assign_blocks(lens_for_tables, n_blocks, gen)
    k_cache, v_cache = _kv_pool((n_blocks, BLOCK, 8, HEAD_DIM), seed, device)
    return dict(q=st["q"], k_cache=k_cache, v_cache=v_cache, context_lens=lens,
                block_tables=table, seq_idx=sel, tail_uncompressed=st["tail_uncompressed"],
                Hq=64, Hk=8)
