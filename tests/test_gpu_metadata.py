"""Per-step metadata built on the GPU vs the oracle's Python loops: bit-exact (integer work).

Follows nanokvllm/engine/model_runner.py:154-219 (prepare_step, prepare_block_tables) and
:265-285 (prepare_decode).
"""
import importlib
import random

import pytest
import torch

from oracle import metadata_ref

pytestmark = pytest.mark.gpu
md_mod = importlib.import_module("nanokv-llm_amd.engine.metadata")
hooks = importlib.import_module("nanokv-llm_amd.engine.compress_hooks")
import sequence as seqmod  # noqa: E402  (test double, tests/sequence.py)
import block_manager as bmmod  # noqa: E402  (test double, tests/block_manager.py)
B = 256
KEYS = ("positions", "slot_mapping", "context_lens", "cu_seqlens_q", "cu_seqlens_k",
        "logits_indices", "block_tables")


def _check(out, ref):
    for key in KEYS:
        assert torch.equal(out[key].cpu(), ref[key]), key
    assert out["max_seqlen_q"] == ref["max_seqlen_q"]
    assert out["max_seqlen_k"] == ref["max_seqlen_k"]


def _random_step(rng, n, max_new, short_tables=False):
    starts, num_new, tables, offs = [], [], [], []
    for _ in range(n):
        start = rng.randrange(0, 20000)
        new = rng.choice([0, 1, 1, 1, rng.randrange(1, max_new + 1)])
        need = (start + new + B - 1) // B
        nb = max(0, need - rng.randrange(0, 3)) if short_tables else need
        tables.append([rng.randrange(0, 100000) for _ in range(nb)])
        starts.append(start)
        num_new.append(new)
        offs.append(rng.choice([0, 0, rng.randrange(0, 50000)]))
    return starts, num_new, tables, offs


@pytest.mark.parametrize("n,max_new,short", [(1, 1, False), (64, 1, False), (37, 3000, False),
                                             (500, 40, True), (3000, 8, True)])
def test_step_metadata_random(dev, n, max_new, short):
    rng = random.Random(n * 7 + max_new)
    starts, num_new, tables, offs = _random_step(rng, n, max_new, short)
    out = md_mod.build_step_metadata(starts, num_new, tables, B, dev, pos_offsets=offs)
    ref = metadata_ref.prepare_step_ref(starts, num_new, tables, B, pos_offsets=offs)
    _check(out, ref)


def test_step_metadata_no_offsets_wide_table_small_blocks(dev):
    rng = random.Random(5)
    starts, num_new, tables, _ = _random_step(rng, 20, 500)
    out = md_mod.build_step_metadata(starts, num_new, tables, 16, dev, bt_width=4096)
    ref = metadata_ref.prepare_step_ref(starts, num_new, tables, 16, width=4096)
    _check(out, ref)


def test_step_metadata_one_long_prompt(dev):
    """A 300k-token prompt: more chunks than the launch's cap, covered by the stride loop."""
    n_tok = 300_000
    tables = [list(range(1000, 1000 + (n_tok + B - 1) // B))]
    out = md_mod.build_step_metadata([0], [n_tok], tables, B, dev)
    ref = metadata_ref.prepare_step_ref([0], [n_tok], tables, B)
    _check(out, ref)


def test_empty_step(dev):
    out = md_mod.build_step_metadata([], [], [], B, dev)
    assert out["cu_seqlens_q"].tolist() == [0] and out["positions"].numel() == 0


def test_hooks_builders_match_oracle(dev):
    """prepare_decode_metadata / prepare_step_metadata on BlockManager-built sequences."""
    bm = bmmod.BlockManager(64, B)
    seqs = []
    for n in (300, 2 * B, 5 * B - 3):
        s = seqmod.Sequence(n)
        bm.allocate(s)
        s.num_computed_tokens = n
        s.append_token()
        bm.may_append(s)
        seqs.append(s)
    seqs[2].rope_pos += 3000  # as after a compression: RoPE runs ahead of the KV length
    md = hooks.prepare_decode_metadata(seqs, B, device=dev)
    ref = metadata_ref.prepare_decode_ref([len(s) for s in seqs], [s.rope_pos for s in seqs],
                                          [s.block_table for s in seqs], B)
    for key in ("positions", "slot_mapping", "context_lens", "block_tables"):
        assert torch.equal(md[key].cpu(), ref[key]), key
    c = seqmod.Sequence(3 * B + 5)
    bm.allocate(c)
    c.num_computed_tokens = 2 * B - 20
    sched = [seqmod.ScheduledSeq(c, 40)] + [seqmod.ScheduledSeq(s, 1) for s in seqs]
    for s in seqs:
        s.num_computed_tokens = len(s) - 1
    st = hooks.prepare_step_metadata(sched, B, device=dev)
    ref = metadata_ref.prepare_step_ref([x.seq.num_computed_tokens for x in sched],
                                        [x.num_new_tokens for x in sched],
                                        [x.seq.block_table for x in sched], B,
                                        pos_offsets=[x.seq.rope_pos - (len(x.seq) - 1)
                                                     for x in sched])
    _check(st, ref)


def test_table_store_across_steps(dev):
    """A serving loop: decode steps append blocks, compression truncates, sequences finish
    and new ones take their rows; the store mode equals the oracle at every step and sends
    only the changed entries."""
    rng = random.Random(9)
    store = md_mod.BlockTableStore(64, 80, dev)
    next_block, next_id = [0], [0]

    def new_seq():
        n = rng.randrange(1, 9000)
        t = list(range(next_block[0], next_block[0] + (n + B - 1) // B))
        next_block[0] += len(t)
        next_id[0] += 1
        return dict(id=next_id[0], len=n, rope=n - 1, table=t)

    live = [new_seq() for _ in range(40)]
    sent_total = 0
    for step in range(30):
        for s in live:  # one decode token each; a new block when the last one is full
            s["len"] += 1
            s["rope"] += 1
            if (s["len"] + B - 1) // B > len(s["table"]):
                s["table"].append(next_block[0])
                next_block[0] += 1
        if step % 7 == 3:  # compression of two sequences: drop middle tokens, free tail blocks
            for s in rng.sample(live, 2):
                if s["len"] > 5 * B:
                    s["len"] -= 3 * B + rng.randrange(0, B)
                    s["table"] = s["table"][:(s["len"] + B - 1) // B]
        if step % 5 == 4:  # two finish, three arrive
            for s in rng.sample(live, 2):
                live.remove(s)
                store.release(s["id"])
            live += [new_seq() for _ in range(3)]
        args = ([s["len"] - 1 for s in live], [1] * len(live), [s["table"] for s in live], B)
        offs = [s["rope"] - (s["len"] - 1) for s in live]
        before = {k: list(v) for k, v in store._sent.items()}
        out = md_mod.build_step_metadata(*args, dev, pos_offsets=offs, store=store,
                                         seq_ids=[s["id"] for s in live])
        ref = metadata_ref.prepare_step_ref(*args, pos_offsets=offs)
        _check(out, ref)
        sent_total += sum(len(s["table"]) for s in live
                          if before.get(s["id"]) != s["table"])
    # far fewer entries were sent than 30 steps x all tables
    assert sent_total < 0.2 * 30 * sum(len(s["table"]) for s in live)


def test_table_store_rejects_long_tables(dev):
    store = md_mod.BlockTableStore(4, 8, dev)
    with pytest.raises(ValueError):
        md_mod.build_step_metadata([0], [1], [list(range(9))], B, dev, store=store, seq_ids=[1])
