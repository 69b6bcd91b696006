"""ORACLE (test infrastructure): the per-step metadata builders, as Python loops on the CPU.

Only tests, the smoke check and the bench's CPU baseline use this module; the
product path never imports it.

Follows ModelRunner.prepare_block_tables and prepare_step,
nanokvllm/engine/model_runner.py:154-158 and :160-219 (per scheduled sequence:
positions range(start, end), slot = block_table[pos // B] * B + pos % B,
cu_seqlens_q/k prefix sums of the new tokens and of end, context_lens = end,
logits_indices = last row of each sequence), and the decode builder of
prepare_decode, :265-285 (one token at KV position len - 1, RoPE position
rope_pos). Two documented differences: a RoPE offset per sequence
(rope_pos - (len - 1), 0 unless the sequence was compressed) is added to the
positions, and a position whose block the table does not hold gets slot -1
where the reference would raise IndexError.
"""
from __future__ import annotations

import torch


def prepare_block_tables_ref(tables: list[list[int]], width: int | None = None) -> torch.Tensor:
    """model_runner.py:154-158: rows right-padded with -1 to the longest (or `width`)."""
    w = max((len(t) for t in tables), default=0) if width is None else width
    return torch.tensor([t[:w] + [-1] * (w - len(t[:w])) for t in tables], dtype=torch.int32
                        ).reshape(len(tables), w)


def prepare_step_ref(starts, num_new, tables, block_size, pos_offsets=None, width=None):
    """model_runner.py:176-198 for sequences s with num_new[s] tokens from KV position starts[s]."""
    positions, slot_mapping, context_lens, logits = [], [], [], []
    cu_q, cu_k = [0], [0]
    max_q = max_k = 0
    for s, (start, n) in enumerate(zip(starts, num_new)):
        end = start + n
        off = pos_offsets[s] if pos_offsets is not None else 0
        positions.extend(p + off for p in range(start, end))
        cu_q.append(cu_q[-1] + n)
        cu_k.append(cu_k[-1] + end)
        max_q, max_k = max(max_q, n), max(max_k, end)
        table = tables[s]
        for pos in range(start, end):
            blk = pos // block_size
            bid = table[blk] if blk < len(table) else -1
            slot_mapping.append(bid * block_size + pos % block_size if bid >= 0 else -1)
        context_lens.append(end)
        logits.append(cu_q[-1] - 1)
    return dict(
        positions=torch.tensor(positions, dtype=torch.int64),
        slot_mapping=torch.tensor(slot_mapping, dtype=torch.int32),
        context_lens=torch.tensor(context_lens, dtype=torch.int32),
        cu_seqlens_q=torch.tensor(cu_q, dtype=torch.int32),
        cu_seqlens_k=torch.tensor(cu_k, dtype=torch.int32),
        logits_indices=torch.tensor(logits, dtype=torch.int64),
        max_seqlen_q=max_q, max_seqlen_k=max_k,
        block_tables=prepare_block_tables_ref(tables, width),
    )


def prepare_decode_ref(lens, rope_pos, tables, block_size):
    """model_runner.py:265-285: one token per sequence at KV position len - 1, RoPE
    position rope_pos, context_lens = len, slot of the last token."""
    return prepare_step_ref([n - 1 for n in lens], [1] * len(lens), tables, block_size,
                            pos_offsets=[r - (n - 1) for r, n in zip(rope_pos, lens)])
