"""Per-step state the decoder attention ops read at call time.

Same fields and functions as vflorence/utils/context.py:6-30.  Here the
tensors live in HBM: ``context_lens``/``block_tables``/``slot_mapping`` are device
tensors built by the runner's step preparation, ``self_metadata`` is a
``hip_attn.SchedulerMetadata`` and each ``cross_staged`` entry is
``(k_cache, v_cache, block_table, seq_lens, SchedulerMetadata)`` for one decoder layer.
Not thread-safe: one forward in flight per process, as in the reference.
"""

from dataclasses import dataclass

import torch


@dataclass(slots=True)
class Context:
    """What one decode step hands every decoder layer's attention ops: the self-attention
    lengths, tables and slots, the query offsets, the self-attention launch metadata,
    the ISA tag and one cross-attention staging tuple per layer."""

    context_lens: torch.Tensor | None = None
    block_tables: torch.Tensor | None = None
    slot_mapping: torch.Tensor | None = None
    query_start_loc: torch.Tensor | None = None
    self_metadata: object | None = None
    isa: str | None = None
    cross_staged: list | None = None


_CONTEXT: Context | None = None


def get_context() -> Context | None:
    """Return the active step's Context (None before the first set_context)."""
    return _CONTEXT


def set_context(**fields) -> None:
    """Publish ``fields`` as the process's Context until the next call; the runner calls
    it with no fields after each step, which leaves an all-None Context."""
    global _CONTEXT
    _CONTEXT = Context(**fields)
