"""Engine hooks of the periodic compression step (host side).

* ``CompressionScheduler.prepare`` -- the compression block of the
  reference's ``ModelRunner.prepare_decode`` (model_runner.py:291-332): a
  decode-step counter fires every ``kv_compress_period`` steps; a sequence is
  eligible iff ``len % B != B-1``, ``tail_uncompressed_len >= W*B`` and it has
  at least W full blocks; the first ``kv_compress_topk`` eligible sequences in
  batch order are selected (``policy="first"``, the reference), or the
  longest ones (``policy="longest"``). It fills the Context fields
  ``is_compress_step``, ``compress_selected_batch_indices``,
  ``compress_selected_seq_ids`` and ``compress_base_context_lens``.
* ``apply_compression_events`` -- ``Scheduler.postprocess``'s event handling
  (scheduler.py:103-125) plus ``BlockManager.truncate_blocks``: dedup by
  batch index, free the tail blocks, ``num_tokens = new_len``,
  ``tail_uncompressed_len = 0``. It also rebases ``num_computed_tokens`` by
  the number of tokens removed, which the reference leaves at the
  uncompressed count (its prepare_step would then index past the truncated
  block table). Events marked skipped (``n_freed = -1`` from the device: a
  selected sequence that was not compressible) change nothing.

Sequences, scheduled items and the block manager are the caller's own objects
(the reference's engine types), read duck-typed: a sequence has ``len()``,
``block_table``, ``seq_id``, ``rope_pos``, ``num_tokens``,
``num_computed_tokens`` and ``tail_uncompressed_len``; a scheduled item is a
sequence or has ``.seq`` and ``.num_new_tokens``; the block manager has
``truncate_blocks(seq, keep_blocks)``.
* ``prepare_decode_metadata`` -- decode metadata as in prepare_decode
  (model_runner.py:265-285): positions = rope_pos, context_lens = physical
  length, slot = last block * B + last_block_num_tokens - 1, block tables
  right-padded with -1; built on the device (engine/metadata.py).
* ``prepare_step_metadata`` -- the mixed prefill/decode builder of
  prepare_step (model_runner.py:160-219), built on the device.
"""
from __future__ import annotations

import torch

from .metadata import BlockTableStore, build_step_metadata


def _seq_of(item):
    """The sequence of a scheduled item (an object with ``.seq``) or the item itself."""
    return getattr(item, "seq", item)


def prepare_block_tables(seqs: list, pad: int = -1) -> list[list[int]]:
    """model_runner.py:154-158 (host lists; the caller moves them to the device)."""
    max_len = max(len(s.block_table) for s in seqs)
    return [s.block_table + [pad] * (max_len - len(s.block_table)) for s in seqs]


def prepare_decode_metadata(seqs: list, block_size: int, device="cuda",
                            store: BlockTableStore | None = None):
    """prepare_decode (model_runner.py:265-285) on the device: one token per sequence at KV
    position len - 1 with RoPE position rope_pos; block tables padded with -1. With a
    ``store`` only the table entries changed since the last step are sent."""
    return build_step_metadata([len(s) - 1 for s in seqs], [1] * len(seqs),
                               [s.block_table for s in seqs], block_size, device,
                               pos_offsets=[s.rope_pos - (len(s) - 1) for s in seqs],
                               store=store, seq_ids=[s.seq_id for s in seqs])


def prepare_step_metadata(scheduled: list, block_size: int, device="cuda",
                          store: BlockTableStore | None = None):
    """prepare_step (model_runner.py:160-219) on the device. Positions carry each sequence's
    RoPE offset (rope_pos - (len - 1)), so a compressed sequence keeps its logical positions
    in a mixed batch too; without compression this is the reference's range(start, end)."""
    seqs = [s.seq for s in scheduled]
    return build_step_metadata([s.num_computed_tokens for s in seqs],
                               [s.num_new_tokens for s in scheduled],
                               [s.block_table for s in seqs], block_size, device,
                               pos_offsets=[s.rope_pos - (len(s) - 1) for s in seqs],
                               store=store, seq_ids=[s.seq_id for s in seqs])


class CompressionScheduler:
    """Decode-step counter + selection of the sequences to compress."""

    def __init__(self, config, policy: str = "first"):
        self.block_size = config.kvcache_block_size
        self.window_blocks = config.kv_compress_window_blocks
        self.topk = config.kv_compress_topk
        self.period = config.kv_compress_period
        self.policy = policy
        self.decode_step_counter = 0

    def select(self, seqs: list) -> tuple[bool, list[int], list[int]]:
        B = self.block_size
        window_tokens = self.window_blocks * B
        self.decode_step_counter += 1
        is_compress_step = self.decode_step_counter % self.period == 0
        selected: list[tuple[int, int]] = []
        if is_compress_step:
            candidates = []
            for i, seq in enumerate(seqs):
                cur = len(seq)
                full_blocks, tail_len = cur // B, cur % B
                if tail_len == B - 1:
                    continue
                if seq.tail_uncompressed_len >= window_tokens and full_blocks >= self.window_blocks:
                    candidates.append((i, seq.seq_id))
            if self.policy == "longest":
                candidates.sort(key=lambda c: (-len(seqs[c[0]]), c[0]))
            selected = candidates[:self.topk]
        return is_compress_step, [x[0] for x in selected], [x[1] for x in selected]

    def prepare(self, context, seqs: list) -> None:
        """Fill the compression fields of ``context`` for this decode step."""
        context.compress_need_mask = None
        context.compress_any = False
        is_step, idx, ids = self.select(seqs)
        context.is_compress_step = is_step
        context.compress_selected_batch_indices = idx
        context.compress_selected_seq_ids = ids
        context.compress_base_context_lens = (context.context_lens.clone()
                                              if is_step and idx else None)


class DeviceCompressionScheduler:
    """The same selection as ``CompressionScheduler`` made on the device
    (nkv_compress_schedule), so a compression step reads no host data and can be captured
    in a HIP graph. The host keeps the step counter (it decides which steps compress, i.e.
    which graph to replay); on a compression step the kernel picks the sequences from the
    device ``context_lens`` and ``tail_uncompressed`` into a -1 padded ``seq_idx`` of
    length topk, which every compression kernel accepts. After the step the last layer's
    events are in ``context.compression_events_device``: pass them to
    ``apply_compression_events_device``."""

    def __init__(self, config, max_batch: int, device, policy: str = "first"):
        self.block_size = config.kvcache_block_size
        self.window_blocks = config.kv_compress_window_blocks
        self.topk = config.kv_compress_topk
        self.period = config.kv_compress_period
        self.policy = policy
        self.step_counter = 0
        i32 = dict(dtype=torch.int32, device=device)
        self.device_counter = torch.zeros(1, **i32)
        self.seq_idx = torch.full((self.topk,), -1, **i32)
        self.n_selected = torch.zeros(1, **i32)
        self.base_context_lens = torch.zeros(max_batch, **i32)

    def prepare(self, context, tail_uncompressed: torch.Tensor) -> bool:
        """Fill the compression fields of ``context``; ``tail_uncompressed`` is a device int32
        [batch] (tokens since each sequence's last compression). Returns is_compress_step."""
        from ..layers.compress_utils import compress_schedule
        context.compress_need_mask = None
        context.compress_any = False
        self.step_counter += 1
        fire = self.step_counter % self.period == 0
        context.is_compress_step = fire
        context.compress_selected_batch_indices = None
        context.compress_selected_seq_ids = None
        context.compression_events_device = None
        if not fire:
            context.compress_seq_idx = None
            context.compress_base_context_lens = None
            return False
        bs = context.context_lens.numel()
        base = self.base_context_lens[:bs]
        compress_schedule(context.context_lens, tail_uncompressed, self.block_size,
                          self.window_blocks, self.topk, 1, self.device_counter, self.seq_idx,
                          self.n_selected, base, policy=self.policy)
        context.compress_seq_idx = self.seq_idx
        context.compress_base_context_lens = base
        return True


def apply_compression_events_device(scheduled: list, events: torch.Tensor | None,
                                    block_manager) -> None:
    """Read the event rows a device-selected step left on the device (one copy) and apply
    them like ``apply_compression_events``; padding rows (batch index -1) are skipped."""
    if events is None:
        return
    from ..layers.compress_utils import events_to_dicts
    apply_compression_events(scheduled, events_to_dicts(events, -1), block_manager)


def apply_compression_events(scheduled: list, events: list[dict] | None, block_manager) -> None:
    """Apply the last layer's events to the host state (scheduler.py:104-125)."""
    if not events:
        return
    dedup = {}
    for ev in events:
        bidx = ev["batch_index"]
        if 0 <= bidx < len(scheduled) and not ev.get("skipped", False):
            dedup[bidx] = ev
    for bidx, ev in dedup.items():
        seq = _seq_of(scheduled[bidx])
        removed = len(seq) - ev["new_context_len"]
        block_manager.truncate_blocks(seq, ev["keep_blocks"])
        seq.num_tokens = ev["new_context_len"]
        seq.num_computed_tokens = max(0, seq.num_computed_tokens - removed)
        seq.tail_uncompressed_len = ev.get("tail_uncompressed_len_after", 0)
