"""The reference's block-manager API (vflorence/engine/block_manager.py:4-73) over the
native block pool (``vfl_pool``, include/vfl_engine.h).

The pool keeps every block's holder count and the free list; this class applies its
decisions to ``Sequence.block_table`` lists.  Same observable behaviour as the
reference: blocks leave the free list from the front and return to its back, a
released table returns its blocks last block first, a fork shares its parent's
blocks, and a sequence about to write into a block others still hold moves to a
fresh copy (the pair is returned for the caller to copy) unless it is the last
holder.  The engine uses the pool directly from its host core; this class serves
code that drives sequences itself (the synthetic beam schedule of the benchmark,
tests) and, over the engine's own pool (``BlockManager.view``), inspection.
"""

from __future__ import annotations

import numpy as np

from .core import BlockPool

_APPEND, _COPY = 1, 2


class BlockManager:
    def __init__(self, num_blocks: int, block_size: int, *, pool: BlockPool | None = None):
        self.pool = pool if pool is not None else BlockPool(num_blocks, block_size)
        self.block_size = block_size

    @classmethod
    def view(cls, pool: BlockPool) -> "BlockManager":
        """Read access to a pool another owner drives (its counts and free list)."""
        return cls(0, pool.block_size, pool=pool)

    @property
    def num_blocks(self) -> int:
        return self.pool.num_blocks

    @property
    def num_free_blocks(self) -> int:
        return self.pool.num_free

    @property
    def ref_counts(self) -> list[int]:
        return self.pool.refcounts().tolist()

    @property
    def free_block_ids(self) -> list[int]:
        """The free list, next block out first."""
        return self.pool.free_list().tolist()

    def reset(self) -> None:
        """Every block free again (after an aborted batch)."""
        self.pool.reset()

    def required_new_blocks(self, seqs) -> int:
        """Blocks that giving every sequence a writable slot would take: one per sequence
        starting a new block, and one per writer of a shared block except its last
        holder."""
        bs = self.block_size
        writes = np.full(len(seqs), -1, dtype=np.int32)
        for i, seq in enumerate(seqs):
            idx = seq.num_cached_tokens // bs
            if idx < len(seq.block_table):
                writes[i] = seq.block_table[idx]
        return self.pool.blocks_needed(writes)

    def ensure_capacity(self, seq) -> tuple[int, int] | None:
        """Make the position ``seq.num_cached_tokens`` writable; returns the (src, dst)
        pair to copy when ``seq`` moved off a shared block, else None."""
        action, block, src = self.pool.prepare_write(seq.block_table, seq.num_cached_tokens)
        if action == _APPEND:
            seq.block_table.append(block)
        elif action == _COPY:
            seq.block_table[seq.num_cached_tokens // self.block_size] = block
            return src, block
        return None

    def fork(self, parent, child) -> None:
        """``child`` shares every block of ``parent``."""
        child.block_table = list(parent.block_table)
        self.pool.share(child.block_table)

    def deallocate(self, seq) -> None:
        """``seq`` lets go of its blocks (last first); blocks nobody holds become free."""
        self.pool.release(seq.block_table)
        seq.block_table.clear()
