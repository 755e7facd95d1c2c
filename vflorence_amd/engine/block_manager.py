"""Paged KV-block allocator with reference counts and copy-on-write.

Same allocation semantics as vflorence/engine/block_manager.py:4-73, so a run
reproduces the reference's block tables and copy pairs exactly: blocks leave a FIFO
free list from the front and return to its back (deallocation walks a table from
its last block), a forked sequence shares every block of its parent, and the
sequence about to write into a shared block gets a private copy -- except the last
holder, which writes in place.  The tables it produces feed the GPU kernels; the
allocator itself stays on the host.
"""

from __future__ import annotations

from collections import deque


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int):
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.reset()

    def reset(self) -> None:
        """Return every block to the free list (after an aborted batch)."""
        self.ref_counts = [0] * self.num_blocks
        self.free_block_ids = deque(range(self.num_blocks))

    @property
    def num_free_blocks(self) -> int:
        return len(self.free_block_ids)

    def _allocate_block(self) -> int:
        if not self.free_block_ids:
            raise RuntimeError("KV cache is full; increase num_blocks")
        block = self.free_block_ids.popleft()
        self.ref_counts[block] = 1
        return block

    def _write_block_index(self, seq) -> int:
        return seq.num_cached_tokens // self.block_size

    def required_new_blocks(self, seqs) -> int:
        """Blocks this step needs: one per sequence entering a new block, plus one per
        sequence writing into a block still shared with a sequence that writes later
        (the last writer of a shared block keeps it)."""
        needed = 0
        holders_left: dict[int, int] = {}
        for seq in seqs:
            idx = self._write_block_index(seq)
            if idx >= len(seq.block_table):
                needed += 1
                continue
            block = seq.block_table[idx]
            refs = holders_left.get(block, self.ref_counts[block])
            if refs > 1:
                needed += 1
                holders_left[block] = refs - 1
        return needed

    def ensure_capacity(self, seq) -> tuple[int, int] | None:
        """Give ``seq`` a writable slot for its next token.

        Appends a fresh block when the token starts one; when the block it writes into
        is shared, moves ``seq`` to a private copy and returns ``(src, dst)`` for the
        caller to copy before the write.  Otherwise returns None.
        """
        idx = self._write_block_index(seq)
        if idx >= len(seq.block_table):
            seq.block_table.append(self._allocate_block())
            return None
        block = seq.block_table[idx]
        if self.ref_counts[block] == 1:
            return None
        private = self._allocate_block()
        self.ref_counts[block] -= 1
        seq.block_table[idx] = private
        return block, private

    def fork(self, parent, child) -> None:
        """``child`` shares all of ``parent``'s blocks."""
        child.block_table = list(parent.block_table)
        for block in child.block_table:
            self.ref_counts[block] += 1

    def deallocate(self, seq) -> None:
        """Drop ``seq``'s references (last block first); unreferenced blocks are freed."""
        for block in reversed(seq.block_table):
            self.ref_counts[block] -= 1
            if self.ref_counts[block] == 0:
                self.free_block_ids.append(block)
        seq.block_table.clear()
