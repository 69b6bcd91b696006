"""Host-side engine hooks of the compression path (CPU): selection, event application,
block bookkeeping and metadata builders, on hand-built sequence states.

Follows nanokvllm/engine/model_runner.py:154-219, 265-332, scheduler.py:103-125,
block_manager.py:94-138 and sequence.py:82-94.
"""
import importlib
import math
from types import SimpleNamespace

import pytest
import torch

from oracle import metadata_ref
from oracle.compress_ref import compress_compact_ref, compress_schedule_ref

hooks = importlib.import_module("nanokv-llm_amd.engine.compress_hooks")
import sequence as seqmod  # noqa: E402  (test double, tests/sequence.py)
import block_manager as bmmod  # noqa: E402  (test double, tests/block_manager.py)
Sequence, ScheduledSeq = seqmod.Sequence, seqmod.ScheduledSeq
BlockManager = bmmod.BlockManager
B, W = 256, 4


def _cfg(period=3, topk=2):
    return SimpleNamespace(kvcache_block_size=B, kv_compress_window_blocks=W,
                           kv_compress_topk=topk, kv_compress_period=period,
                           kv_compress_keep_blocks=2, kv_compress_keep_extra_tokens=1)


def _seq(n, tail_uncompressed=None, seq_id=None):
    s = Sequence(n, seq_id=seq_id)
    s.tail_uncompressed_len = n if tail_uncompressed is None else tail_uncompressed
    return s


def test_selection_period_and_rules():
    sched = hooks.CompressionScheduler(_cfg(period=3, topk=2))
    seqs = [
        _seq(5 * B + (B - 1), seq_id=10),  # tail == B-1: skipped
        _seq(3 * B + 7, seq_id=11),        # only 3 full blocks: skipped
        _seq(6 * B + 3, tail_uncompressed=W * B - 1, seq_id=12),  # too little new data
        _seq(4 * B, seq_id=13),            # exactly W full blocks, tail 0: eligible
        _seq(9 * B + 100, seq_id=14),      # eligible
        _seq(7 * B + 1, seq_id=15),        # eligible, but topk = 2 takes the first two
    ]
    fired = []
    for step in range(1, 7):
        is_step, idx, ids = sched.select(seqs)
        fired.append(is_step)
        if is_step:
            assert idx == [3, 4] and ids == [13, 14]
        else:
            assert idx == [] and ids == []
    assert fired == [False, False, True, False, False, True]


def test_selection_longest_policy_and_context_fields():
    sched = hooks.CompressionScheduler(_cfg(period=1, topk=2), policy="longest")
    seqs = [_seq(4 * B + 1), _seq(9 * B + 5), _seq(6 * B), _seq(9 * B + 5)]
    ctx = SimpleNamespace(context_lens=torch.tensor([len(s) for s in seqs], dtype=torch.int32))
    sched.prepare(ctx, seqs)
    assert ctx.is_compress_step
    assert ctx.compress_selected_batch_indices == [1, 3]  # longest, ties by batch order
    assert torch.equal(ctx.compress_base_context_lens, ctx.context_lens)
    assert ctx.compress_base_context_lens is not ctx.context_lens  # a snapshot


def test_block_manager_append_and_truncate():
    bm = BlockManager(16, B)
    s = _seq(2 * B)
    bm.allocate(s)
    assert len(s.block_table) == 2 and len(bm.free_block_ids) == 14
    s.append_token()  # len % B == 1: a new block
    assert bm.can_append(s)
    bm.may_append(s)
    assert len(s.block_table) == 3
    for _ in range(B - 1):
        s.append_token()
        bm.may_append(s)
    assert len(s) == 3 * B and bm.blocks[s.block_table[-1]].hash != -1  # sealed when full
    freed = s.block_table[2:]
    bm.truncate_blocks(s, 2)
    assert s.block_table and len(s.block_table) == 2
    assert all(b in bm.free_block_ids for b in freed)
    assert bm.blocks[s.block_table[-1]].hash == -1  # the kept last block is writable again


def _compress_on_cpu(seqs, bm, selected, keep=2 * B + 1):
    """One compression step's events from the oracle (one layer), on a zero cache."""
    n_blocks = len(bm.blocks)
    kc = torch.zeros(n_blocks, B, 1, 128, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    bt = torch.tensor(hooks.prepare_block_tables(seqs), dtype=torch.int32)
    base = torch.tensor([len(s) for s in seqs], dtype=torch.int32)
    ctx = base.clone()
    keep_idx = torch.arange(keep).view(1, 1, keep).expand(len(selected), 1, keep).clone()
    ok, _, events = compress_compact_ref(None, kc, vc, bt, base, ctx, selected, B, W, 2, 1, 0, 1,
                                         keep_idx=keep_idx)
    assert ok
    return events, ctx


@pytest.mark.parametrize("tail", [0, 37, B - 2])
def test_events_apply_and_decoding_continues(tail):
    """Events free exactly the reported blocks; the sequence keeps appending across the
    next block boundary (may_append's seal asserts hold); num_computed_tokens rebases."""
    bm = BlockManager(64, B)
    seqs = [_seq(5 * B + tail, seq_id=0), _seq(3 * B + 9, seq_id=1), _seq(8 * B + tail, seq_id=2)]
    for s in seqs:
        bm.allocate(s)
        s.num_computed_tokens = len(s)
    sched = hooks.CompressionScheduler(_cfg(period=1, topk=3))
    _, idx, _ = sched.select(seqs)
    assert idx == [0, 2]
    events, ctx = _compress_on_cpu(seqs, bm, idx)
    before_free = set(bm.free_block_ids)
    old = [len(s) for s in seqs]
    scheduled = [ScheduledSeq(s, 1) for s in seqs]
    hooks.apply_compression_events(scheduled, events + events[:1], bm)  # duplicate: deduped
    for ev in events:
        s = seqs[ev["batch_index"]]
        assert len(s) == ev["new_context_len"] == old[ev["batch_index"]] - W * B + 2 * B + 1
        assert len(s.block_table) == ev["keep_blocks"] == (len(s) + B - 1) // B
        assert s.num_computed_tokens == len(s) and s.tail_uncompressed_len == 0
        assert set(ev["freed_block_ids"]) <= set(bm.free_block_ids) - before_free
        assert len(ev["freed_block_ids"]) == (1 if tail == 0 else 2)
    assert len(seqs[1]) == old[1] and int(ctx[1]) == old[1]
    # decoding continues: append through the next block boundary
    for s in seqs:
        for _ in range(B + 3):
            s.append_token()
            assert bm.can_append(s)
            bm.may_append(s)
        assert len(s.block_table) == (len(s) + B - 1) // B


def test_decode_and_step_metadata():
    """The metadata oracle (model_runner.py:154-219, 265-285) on hand-built states; the
    device builders are held to it in tests/test_gpu_metadata.py."""
    bm = BlockManager(32, B)
    a, b = _seq(300), _seq(2 * B)
    for s in (a, b):
        bm.allocate(s)
    a.num_computed_tokens, b.num_computed_tokens = 300, 2 * B
    b.append_token()
    bm.may_append(b)
    md = metadata_ref.prepare_decode_ref([len(a), len(b)], [a.rope_pos, b.rope_pos],
                                         [a.block_table, b.block_table], B)
    assert md["context_lens"].tolist() == [300, 2 * B + 1]
    assert md["slot_mapping"].tolist() == [a.block_table[1] * B + 300 - B - 1, b.block_table[2] * B]
    assert md["block_tables"].tolist() == [a.block_table + [-1], b.block_table]
    assert md["positions"].tolist() == [a.rope_pos, b.rope_pos]
    # chunked prefill of 40 new tokens of a fresh prompt next to a 1-token decode
    c = _seq(3 * B + 5)
    bm.allocate(c)
    c.num_computed_tokens = 2 * B - 20
    st = metadata_ref.prepare_step_ref([c.num_computed_tokens, a.num_computed_tokens], [40, 1],
                                       [c.block_table, a.block_table], B)
    assert st["cu_seqlens_q"].tolist() == [0, 40, 41]
    assert st["cu_seqlens_k"].tolist() == [0, 2 * B + 20, 2 * B + 20 + 301]
    assert st["max_seqlen_q"] == 40 and st["max_seqlen_k"] == 2 * B + 20
    assert st["logits_indices"].tolist() == [39, 40]
    pos = list(range(2 * B - 20, 2 * B + 20))
    assert st["positions"].tolist() == pos + [300]
    exp = [c.block_table[p // B] * B + p % B for p in pos] + [a.block_table[300 // B] * B + 300 % B]
    assert st["slot_mapping"].tolist() == exp
    # a compressed sequence keeps its RoPE position; a table too short gives slot -1
    d = metadata_ref.prepare_decode_ref([10], [5000], [[7]], B)
    assert d["positions"].tolist() == [5000] and d["slot_mapping"].tolist() == [7 * B + 9]
    e = metadata_ref.prepare_step_ref([B - 1], [2], [[3]], B)
    assert e["slot_mapping"].tolist() == [3 * B + B - 1, -1]


@pytest.mark.parametrize("policy", ["first", "longest"])
def test_schedule_oracle_matches_host_scheduler(policy):
    """The schedule oracle (what the device kernel is tested against) and the host
    CompressionScheduler make the same choice on random states, firing on the same steps."""
    gen = torch.Generator().manual_seed(3 if policy == "first" else 4)
    sched = hooks.CompressionScheduler(_cfg(period=2, topk=5), policy=policy)
    counter = 0
    for _ in range(6):
        lens = torch.randint(B, 20 * B, (60,), generator=gen).tolist()
        lens[::7] = [(x // B) * B + B - 1 for x in lens[::7]]  # tail == B-1 rows
        tails = torch.randint(0, 2 * W * B, (60,), generator=gen).tolist()
        seqs = [_seq(n, tail_uncompressed=t) for n, t in zip(lens, tails)]
        fired, idx, _ = sched.select(seqs)
        counter, sel, fired_ref = compress_schedule_ref(lens, tails, B, W, 5, counter, 2, policy)
        assert fired == fired_ref and idx == sel
    # a hand-built case: only rows 0 and 2 qualify
    assert compress_schedule_ref([1024, 1279, 2000, 1023, 5000], [1024, 2000, 1024, 5000, 100],
                                 B, W, 2, 2, 3) == (3, [0, 2], True)


def test_device_events_skip_padding_rows():
    """apply_compression_events_device: padding rows (batch index -1) are ignored, real rows
    are applied like the host path's event dicts."""
    bm = BlockManager(32, B)
    a = _seq(6 * B + 10)
    bm.allocate(a)
    n_before = len(bm.free_block_ids)
    ev = torch.full((2, 4 + 8), -1, dtype=torch.int32)
    ev[0, :4] = torch.tensor([-1, 0, 0, 0])
    new_len = 6 * B + 10 - W * B + 513
    keep_blocks = (new_len + B - 1) // B
    freed = a.block_table[keep_blocks:]
    ev[1, :4] = torch.tensor([0, new_len, keep_blocks, len(freed)])
    ev[1, 4:4 + len(freed)] = torch.tensor(freed)
    hooks.apply_compression_events_device([ScheduledSeq(a, 1)], ev, bm)
    assert len(a) == new_len and len(a.block_table) == keep_blocks
    assert a.tail_uncompressed_len == 0 and len(bm.free_block_ids) == n_before + len(freed)


def test_skipped_event_changes_no_host_state():
    """An event row marked skipped (n_freed = -1: the selected sequence was not
    compressible) leaves the sequence and the block manager as they were."""
    import numpy as np
    cu = importlib.import_module("nanokv-llm_amd.layers.compress_utils")
    bm = BlockManager(32, B)
    s0, s1 = _seq(5 * B + 7), _seq(3 * B + 9)
    for s in (s0, s1):
        bm.allocate(s)
    # a compressed row for s0 and a skipped row for s1, as nkv_compress_finalize writes them
    kb = math.ceil((5 * B + 7 - W * B + 2 * B + 1) / B)
    freed = s0.block_table[kb:]
    rows = np.full((2, 4 + 8), -1, dtype=np.int32)
    rows[0, :4] = [0, 5 * B + 7 - W * B + 2 * B + 1, kb, len(freed)]
    rows[0, 4:4 + len(freed)] = freed
    rows[1, :4] = [1, 3 * B + 9, 4, -1]
    evs = cu.events_to_dicts(torch.from_numpy(rows), 0)
    assert evs[1]["skipped"] and "skipped" not in evs[0]
    before = (len(s1), list(s1.block_table), s1.num_computed_tokens, s1.tail_uncompressed_len)
    free_before = len(bm.free_block_ids)
    hooks.apply_compression_events([s0, s1], evs, bm)
    assert (len(s1), list(s1.block_table), s1.num_computed_tokens,
            s1.tail_uncompressed_len) == before
    assert len(s0) == 5 * B + 7 - W * B + 2 * B + 1 and s0.tail_uncompressed_len == 0
    assert len(bm.free_block_ids) == free_before + len(freed)
