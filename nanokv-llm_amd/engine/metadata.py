"""Per-step attention metadata built on the device (libnkv_amd.so).

Replaces the per-token Python loop of ModelRunner.prepare_step and the
padding of prepare_block_tables (nanokvllm/engine/model_runner.py:154-219),
and the decode builder of prepare_decode (:265-285). The host packs one int32
buffer -- per sequence the start (KV position of the first new token), the
number of new tokens, the RoPE offset (rope_pos - (len - 1): 0 unless the
sequence was compressed) and its block table -- copies it to the device once,
and two kernels expand it into positions, slot_mapping, cu_seqlens_q/k,
context_lens, logits_indices and the padded block tables.

Block tables travel either whole (a flat list with offsets), or through a
``BlockTableStore``: a device-resident table per live sequence that the host
keeps current by sending only the entries that changed since the previous
step (a decode step appends one block per sequence every block_size tokens;
compression truncates). Host work is then O(sequences + changed blocks).
"""
from __future__ import annotations

import itertools
import struct

import torch

from .. import _lib

NKV_META_POS_OFFSETS = 1


class BlockTableStore:
    """Device copy of the block tables of up to ``max_seqs`` live sequences, each up to
    ``max_blocks_per_seq`` entries. ``sync`` assigns rows to new sequences and returns the
    (row, col, id) updates that bring the device copy level with the host tables; the
    updates are applied by the next ``build_step_metadata`` on the device stream.
    ``release`` frees a finished sequence's row."""

    def __init__(self, max_seqs: int, max_blocks_per_seq: int, device):
        self.table = torch.full((max_seqs, max_blocks_per_seq), -1, dtype=torch.int32,
                                device=device)
        self.max_blocks = max_blocks_per_seq
        self._free = list(range(max_seqs - 1, -1, -1))
        self._row: dict[int, int] = {}
        self._sent: dict[int, list[int]] = {}

    def release(self, seq_id: int) -> None:
        row = self._row.pop(seq_id, None)
        if row is not None:
            self._sent.pop(seq_id, None)
            self._free.append(row)

    def sync(self, seq_ids: list[int], tables: list[list[int]]):
        """-> (rows, counts, flat updates [row, col, id, ...])."""
        counts = list(map(len, tables))
        if counts and max(counts) > self.max_blocks:
            raise ValueError(f"block table of {max(counts)} entries exceeds the store's "
                             f"{self.max_blocks}")
        row_of, sent_of = self._row, self._sent
        rows = [row_of.get(sid, -1) for sid in seq_ids]
        # decode steps leave almost every table as it was: find the others first
        changed = [i for i, (r, sid, t) in enumerate(zip(rows, seq_ids, tables))
                   if r < 0 or sent_of[sid] != t]
        updates = []
        for i in changed:
            sid, t = seq_ids[i], tables[i]
            row = row_of.get(sid, -1)  # set earlier in this call if sid repeats
            if row < 0:
                if not self._free:
                    raise RuntimeError("BlockTableStore is full: release finished sequences")
                row = self._free.pop()
                row_of[sid] = row
                sent = []
            else:
                sent = sent_of[sid]
            rows[i] = row
            k, lim = 0, min(len(t), len(sent))
            while k < lim and t[k] == sent[k]:
                k += 1
            for c in range(k, len(t)):
                updates += (row, c, t[c])
            sent_of[sid] = list(t)
        return rows, counts, updates


def build_step_metadata(starts: list[int], num_new: list[int], tables: list[list[int]],
                        block_size: int, device, pos_offsets: list[int] | None = None,
                        bt_width: int | None = None, store: BlockTableStore | None = None,
                        seq_ids: list[int] | None = None) -> dict:
    """Metadata of one step for sequences s scheduling num_new[s] tokens from KV position
    starts[s]; returns device tensors plus host ints max_seqlen_q / max_seqlen_k. With a
    ``store`` (and the sequences' ``seq_ids``) only changed table entries are sent."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    _lib.require_device(device, table=store.table if store is not None else None)
    n = len(starts)
    if len(num_new) != n or len(tables) != n or (pos_offsets is not None and len(pos_offsets) != n):
        raise ValueError("starts, num_new, tables (and pos_offsets) need one entry per sequence")
    if n and (min(starts) < 0 or min(num_new) < 0):
        raise ValueError("starts and num_new must be >= 0")
    total = sum(num_new)
    max_q = max(num_new, default=0)
    max_k = max((s + k for s, k in zip(starts, num_new)), default=0)
    width = max((len(t) for t in tables), default=0) if bt_width is None else bt_width
    vals = list(starts)
    vals += num_new
    if pos_offsets is not None:
        vals += pos_offsets
    n_updates = 0
    if store is not None:
        if seq_ids is None or len(seq_ids) != n:
            raise ValueError("a BlockTableStore needs one seq_id per sequence")
        rows, counts, updates = store.sync(seq_ids, tables)
        n_updates = len(updates) // 3
        vals += rows
        vals += counts
        vals += updates
    else:
        vals.append(0)
        vals += itertools.accumulate(map(len, tables))
        vals += itertools.chain.from_iterable(tables)
    # struct converts the Python ints in C (several times faster than numpy or torch from
    # a list); it raises on values outside int32
    try:
        packed_buf = bytearray(struct.pack(f"{len(vals)}i", *vals))
    except struct.error as e:
        raise ValueError(f"step metadata value outside int32: {e}") from None
    i32 = dict(dtype=torch.int32, device=device)
    out = dict(
        positions=torch.empty(total, dtype=torch.int64, device=device),
        slot_mapping=torch.empty(total, **i32),
        context_lens=torch.empty(n, **i32),
        cu_seqlens_q=torch.empty(n + 1, **i32),
        cu_seqlens_k=torch.empty(n + 1, **i32),
        logits_indices=torch.empty(n, dtype=torch.int64, device=device),
        block_tables=torch.empty(n, width, **i32),
        max_seqlen_q=max_q, max_seqlen_k=max_k,
    )
    if n == 0 and n_updates == 0:
        out["cu_seqlens_q"].zero_()
        out["cu_seqlens_k"].zero_()
        return out
    # pinned staging (torch's host allocator keeps it until the copy has run)
    packed = torch.frombuffer(packed_buf, dtype=torch.int32).pin_memory().to(device,
                                                                             non_blocking=True)
    bt = out["block_tables"]
    st = store.table if store is not None else None
    rc = _lib.lib().nkv_build_step_metadata(
        packed.data_ptr(), n, block_size, max_q, total,
        NKV_META_POS_OFFSETS if pos_offsets is not None else 0,
        st.data_ptr() if st is not None else None, st.stride(0) if st is not None else 0,
        st.size(0) if st is not None else 0, n_updates,
        out["cu_seqlens_q"].data_ptr(), out["cu_seqlens_k"].data_ptr(),
        out["context_lens"].data_ptr(), out["positions"].data_ptr(),
        out["slot_mapping"].data_ptr(), out["logits_indices"].data_ptr(), None,
        bt.data_ptr() if width else None, max(width, 1), width,
        _lib.stream_of(out["positions"]))
    _lib.check(rc, "build_step_metadata")
    return out
