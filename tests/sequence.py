"""TEST DOUBLE: the per-request state the attention path reads (host bookkeeping).

Used by the tests to drive the engine hooks; the package reads these fields
duck-typed from the caller's own sequence objects and ships no Sequence.

Keeps the fields of nanokvllm/engine/sequence.py:15-94 that the compression
path depends on: ``num_tokens`` is the PHYSICAL cache length (shrinks after
compression), ``rope_pos`` the logical position (never shrinks) and
``tail_uncompressed_len`` the tokens appended since the last compression.
Token ids are not kept: nothing on this path reads them.
"""
from __future__ import annotations

from dataclasses import dataclass
from itertools import count


class Sequence:
    block_size = 256
    counter = count()

    def __init__(self, num_prompt_tokens: int, seq_id: int | None = None):
        self.seq_id = next(Sequence.counter) if seq_id is None else seq_id
        self.num_tokens = num_prompt_tokens
        self.num_prompt_tokens = num_prompt_tokens
        self.num_cached_tokens = 0
        self.num_computed_tokens = 0
        self.block_table: list[int] = []
        self.rope_pos = num_prompt_tokens - 1
        self.tail_uncompressed_len = 0
        self.generated_completion_tokens = 0

    def __len__(self):
        return self.num_tokens

    @property
    def is_prefill_done(self) -> bool:
        return self.num_computed_tokens >= self.num_prompt_tokens

    @property
    def num_blocks(self) -> int:
        return (self.num_tokens + self.block_size - 1) // self.block_size

    @property
    def last_block_num_tokens(self) -> int:
        return self.num_tokens - (self.num_blocks - 1) * self.block_size

    def append_token(self) -> None:
        """sequence.py:82-94: one more token in cache order and in RoPE order."""
        self.num_tokens += 1
        self.generated_completion_tokens += 1
        self.rope_pos += 1
        self.tail_uncompressed_len += 1


@dataclass
class ScheduledSeq:
    seq: Sequence
    num_new_tokens: int
