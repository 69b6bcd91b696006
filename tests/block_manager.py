"""TEST DOUBLE: Paged block allocator for the K/V pool (host bookkeeping, no prefix cache).

Follows the allocation, append and release rules of
nanokvllm/engine/block_manager.py:38-138 that the attention path depends on:
a sequence owns ``ceil(len / B)`` blocks, a new block is taken when
``len % B == 1`` after an append, and ``truncate_blocks`` releases the tail
blocks freed by a compression step. Prefix hashing (xxhash) is not kept; a
block is "sealed" (hash != -1) once full, which is all ``may_append`` checks.
The package takes the caller's own block manager (any object with
``truncate_blocks(seq, keep_blocks)``).
"""
from __future__ import annotations

from collections import deque

from sequence import Sequence


class Block:
    def __init__(self, block_id: int):
        self.block_id = block_id
        self.ref_count = 0
        self.hash = -1


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        self.block_size = block_size
        self.blocks = [Block(i) for i in range(num_blocks)]
        self.free_block_ids: deque[int] = deque(range(num_blocks))
        self.used_block_ids: set[int] = set()

    def _allocate_block(self, block_id: int) -> Block:
        block = self.blocks[block_id]
        assert block.ref_count == 0
        block.ref_count = 1
        block.hash = -1
        self.free_block_ids.remove(block_id)
        self.used_block_ids.add(block_id)
        return block

    def _deallocate_block(self, block_id: int) -> None:
        assert self.blocks[block_id].ref_count == 0
        self.used_block_ids.remove(block_id)
        self.free_block_ids.append(block_id)

    def can_allocate(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= seq.num_blocks

    def allocate(self, seq: Sequence) -> None:
        assert not seq.block_table
        for i in range(seq.num_blocks):
            block = self._allocate_block(self.free_block_ids[0])
            if (i + 1) * self.block_size <= seq.num_tokens:
                block.hash = i  # full block: sealed
            seq.block_table.append(block.block_id)

    def deallocate(self, seq: Sequence) -> None:
        for block_id in reversed(seq.block_table):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.num_cached_tokens = 0
        seq.block_table.clear()

    def can_append(self, seq: Sequence) -> bool:
        return len(self.free_block_ids) >= (len(seq) % self.block_size == 1)

    def may_append(self, seq: Sequence) -> None:
        """Called after the new token is counted in len(seq) (block_manager.py:94-113)."""
        last = self.blocks[seq.block_table[-1]]
        if len(seq) % self.block_size == 1:
            assert last.hash != -1
            block = self._allocate_block(self.free_block_ids[0])
            seq.block_table.append(block.block_id)
        elif len(seq) % self.block_size == 0:
            assert last.hash == -1
            last.hash = len(seq.block_table) - 1
        else:
            assert last.hash == -1

    def truncate_blocks(self, seq: Sequence, keep_blocks: int) -> None:
        """Release seq.block_table[keep_blocks:] (block_manager.py:117-138)."""
        if keep_blocks >= len(seq.block_table):
            return
        for block_id in reversed(seq.block_table[keep_blocks:]):
            block = self.blocks[block_id]
            block.ref_count -= 1
            if block.ref_count == 0:
                self._deallocate_block(block_id)
        seq.block_table = seq.block_table[:keep_blocks]
        seq.num_cached_tokens = min(seq.num_cached_tokens, keep_blocks * self.block_size)
        if seq.block_table:
            self.blocks[seq.block_table[-1]].hash = -1
