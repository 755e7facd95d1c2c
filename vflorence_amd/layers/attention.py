"""Decoder attention custom ops backed by the gfx950 kernels.

Drop-in for vflorence/layers/attention.py: the two opaque ``torch.library`` ops keep
their names, schemas, mutation annotations and fakes
(``vflorence::self_attention`` :42-85, ``vflorence::cross_attention`` :88-115), and
``stage_cross`` (:9-39) keeps its arguments and per-layer tuple layout, so model code
and ``torch.compile`` of the decoder are unchanged.  The op bodies read the step's
Context at call time and enqueue HIP kernels on the current stream; nothing runs on
the CPU.
"""

from __future__ import annotations

import numpy as np
import torch

from .. import hip_attn
from .._lib import check, lib
from ..utils.context import get_context

# Head sizes with a gfx950 kernel (the reference lists its CPU ISAs' sizes at :6).
HEAD_DIMS = set(hip_attn.SUPPORTED_HEAD_DIMS)


def beam_groups(pages, enc_lens, max_group: int = hip_attn.MAX_GROUP_SIZE) -> list[int]:
    """Start offsets of runs of consecutive rows that read the same encoder pages.

    The runner repeats one page tensor for every beam of a request and keeps a
    request's beams adjacent (vflorence/engine/scheduler.py:121-126), so a run is one
    request.  Runs are cut at ``max_group`` rows.  Returns ``[0, ..., len(pages)]``.
    """
    starts = [0]
    for i in range(1, len(pages)):
        same = enc_lens[i] == enc_lens[i - 1] and (
            pages[i] is pages[i - 1]
            or (pages[i].shape == pages[i - 1].shape and torch.equal(pages[i], pages[i - 1]))
        )
        if not same or i - starts[-1] >= max_group:
            starts.append(i)
    starts.append(len(pages))
    return starts


class CrossStagingBuffers:
    """Fixed-address staging for ``stage_cross``: a pinned host buffer and its device
    twin laid out for up to ``max_rows`` rows and ``max_pages`` pages per row.

    int32 words: lengths [max_rows] | group starts [max_rows + 1] | dispatch order
    [max_rows] | page table [max_rows, max_pages] | (16-byte aligned) one slot
    descriptor per launch slot (``hip_attn.build_slot_descriptors``: the slot's group,
    length and page row, which the launch reads in one load level).  Every batch of n
    rows uses the
    same addresses and launch shape (a group slot count fixed per row count and beam
    width, unused slots marked -1 in the order),
    so a decode step captured in a HIP graph stays valid when the batch's requests,
    and hence its beam groups and pages, change.
    """

    def __init__(self, max_rows: int, max_pages: int, device):
        self.max_rows, self.max_pages = max_rows, max_pages
        m = max_rows
        self.desc_stride = hip_attn.slot_descriptor_stride(max_pages)
        desc_at = (3 * m + 1 + m * max_pages + 3) // 4 * 4
        words = desc_at + m * self.desc_stride
        self.host = torch.zeros(words, dtype=torch.int32, pin_memory=True)
        self.dev = torch.zeros(words, dtype=torch.int32, device=device)
        self.copied = torch.cuda.Event()
        self.copied.record()
        self.np = self.host.numpy()
        self.offsets = (0, m, 2 * m + 1, 3 * m + 1, desc_at)

    def views(self, n: int, slots: int | None = None):
        """Lengths and table of ``n`` rows; group starts, order and slot descriptors of
        ``slots`` launch slots (default ``n``)."""
        o, g = self.offsets, n if slots is None else slots
        desc = hip_attn.GroupPlan(self.dev[o[4]: o[4] + g * self.desc_stride], self.desc_stride,
                                  g, self.max_pages)
        return (self.dev[o[0]: o[0] + n], self.dev[o[1]: o[1] + g + 1], self.dev[o[2]: o[2] + g],
                self.dev[o[3]: o[3] + self.max_rows * self.max_pages]
                .view(self.max_rows, self.max_pages)[:n], desc)


def _stage_into(buffers: CrossStagingBuffers, pages, enc_lens, starts, run, slots=None):
    n = len(pages)
    if n > buffers.max_rows or max(len(p) for p in pages) > buffers.max_pages:
        raise ValueError(f"{n} rows / {max(len(p) for p in pages)} pages exceed the staging "
                         f"capacity ({buffers.max_rows} rows, {buffers.max_pages} pages)")
    ng = len(starts) - 1
    o, h = buffers.offsets, buffers.np
    buffers.copied.synchronize()  # the previous upload has left the host buffer
    h[o[0]: o[0] + n] = enc_lens
    h[o[1]: o[1] + ng + 1] = starts
    h[o[1] + ng + 1: o[1] + n + 1] = n  # empty groups past the last
    order = hip_attn.balanced_order([enc_lens[a] for a in starts[:-1]], run)
    h[o[2]: o[2] + ng] = order
    h[o[2] + ng: o[2] + n] = -1  # their workgroups exit at once
    table = h[o[3]: o[3] + buffers.max_rows * buffers.max_pages].reshape(
        buffers.max_rows, buffers.max_pages)
    _fill_page_table(table, pages)
    base = buffers.host.data_ptr()
    g = n if slots is None else slots
    check(lib.vfl_build_slot_descriptors(
        base + 4 * o[3], buffers.max_pages, buffers.max_pages, base + 4 * o[0], n,
        base + 4 * o[1], base + 4 * o[2], ng, base + 4 * o[4], g, buffers.desc_stride))
    # the parts the launches read: lengths, starts, order and the n table rows, then the
    # g slot descriptors
    end, d0, d1 = o[3] + n * buffers.max_pages, o[4], o[4] + g * buffers.desc_stride
    buffers.dev[:end].copy_(buffers.host[:end], non_blocking=True)
    buffers.dev[d0:d1].copy_(buffers.host[d0:d1], non_blocking=True)
    buffers.copied.record()
    return buffers.views(n, slots)


def _fill_page_table(table: np.ndarray, pages) -> None:
    """Rows 0 .. len(pages) - 1 of ``table`` hold each row's pages, zero-padded: one
    scatter of all rows' pages (a row list that repeats one page array or tensor per
    beam converts it once)."""
    n = len(pages)
    arrays, seen = [], {}
    for p in pages:
        a = seen.get(id(p))
        if a is None:
            a = p if isinstance(p, np.ndarray) else (
                p.numpy() if isinstance(p, torch.Tensor) else np.asarray(p, dtype=np.int32))
            seen[id(p)] = a
        arrays.append(a)
    counts = np.fromiter(map(len, arrays), dtype=np.int64, count=n)
    table[:n] = 0
    total = int(counts.sum())
    if total:
        rows = np.repeat(np.arange(n), counts)
        cols = np.arange(total) - np.repeat(np.cumsum(counts) - counts, counts)
        table[rows, cols] = np.concatenate(arrays)


def stage_cross(layers, pages, enc_lens, block_size: int, isa: str, *, buffers=None,
                slots=None, group_starts=None):
    """Point this step's sequences at their encoder K/V pages in each layer's pool.

    ``pages[i]`` (int32 tensor) and ``enc_lens[i]`` belong to running sequence i; beams
    of one request repeat its pages.  Nothing is copied: the padded block table,
    lengths and beam groups go to the device once and every layer shares them.
    With ``buffers`` (a ``CrossStagingBuffers``) they go to its fixed addresses
    instead of a fresh allocation, with ``slots`` launch slots (one per row when not
    given, or when the rows form more groups than that), the unused ones exiting at
    once.  With ``buffers``, ``pages[i]`` may also be an int32 numpy array, and a caller
    that knows the rows' requests passes ``group_starts`` (``beam_groups``' result for
    these rows: runs of rows sharing pages, cut at 8) instead of having the pages
    compared.
    """
    attn = layers[0].encoder_attn
    device = attn.k_cache.device
    if group_starts is not None and buffers is None:
        raise ValueError("group_starts is for staging into CrossStagingBuffers")
    if group_starts is None:
        starts = beam_groups(pages, enc_lens)
    else:
        gs = np.asarray(group_starts, dtype=np.int64)
        steps = np.diff(gs)
        if (gs.ndim != 1 or gs.size < 2 or gs[0] != 0 or gs[-1] != len(pages)
                or (steps <= 0).any() or (steps > hip_attn.MAX_GROUP_SIZE).any()):
            raise ValueError(f"group_starts must rise from 0 to {len(pages)} in runs of 1 to "
                             f"{hip_attn.MAX_GROUP_SIZE} rows")
        starts = gs.tolist()
    max_group = max(b - a for a, b in zip(starts, starts[1:]))
    n, ng = len(pages), len(starts) - 1
    # every (group, head) workgroup is resident at once: balance long and short groups
    # over the CUs (hip_attn.balanced_order)
    run = hip_attn.resident_run(device, attn.num_heads) if device.type == "cuda" else 1
    active = None
    if buffers is not None:
        if slots is None or not ng <= slots <= n:
            slots = n
        seq_lens, group_start, group_order, block_table, desc = _stage_into(
            buffers, pages, enc_lens, starts, run, slots)
        # n slots, about n / (beams per request) of them working: waves per workgroup as
        # for a launch of that many groups (4 beams of 64 requests: 1024 workgroups and
        # eight waves, not the 4096 slots' four).  Slots over beam width, not the exact
        # group count, so every batch of one row bucket and beam width launches alike.
        # (padding rows share one empty page list and group together: not counted)
        beams = max((b - a for a, b in zip(starts, starts[1:]) if enc_lens[a] > 0), default=1)
        active = -(-n // beams)
        max_group = hip_attn.MAX_GROUP_SIZE  # one launch shape for every batch of n rows
    else:
        block_table = torch.nn.utils.rnn.pad_sequence(
            [p.to(torch.int32).cpu() for p in pages], batch_first=True
        )
        width = block_table.shape[1]
        order = hip_attn.balanced_order([enc_lens[a] for a in starts[:-1]], run)
        lens_h = torch.tensor(enc_lens, dtype=torch.int32)
        starts_h = torch.tensor(starts, dtype=torch.int32)
        order_h = torch.tensor(order, dtype=torch.int32)
        parts = [lens_h, starts_h, order_h, block_table.flatten()]
        fixed = sum(t.numel() for t in parts)
        if max_group > 1:  # slot descriptors, 16-byte aligned after the rest
            desc_h = hip_attn.build_slot_descriptors(block_table, lens_h, starts_h,
                                                     group_order=order_h)
            parts += [torch.zeros(-fixed % 4, dtype=torch.int32), desc_h.words]
        # One host->device copy: [seq_lens (n) | group starts (ng + 1) | group order (ng) |
        # block table (n * width) | slot descriptors].
        dev = torch.cat(parts).to(device)
        seq_lens = dev[:n]
        group_start = dev[n : n + ng + 1] if max_group > 1 else None
        group_order = dev[n + ng + 1 : n + 2 * ng + 1]
        block_table = dev[n + 2 * ng + 1 : fixed].view(n, width)
        desc = None
        if max_group > 1:
            at = fixed + (-fixed % 4)
            desc = hip_attn.GroupPlan(dev[at: at + desc_h.words.numel()], desc_h.stride,
                                      desc_h.slots, desc_h.max_blocks)
    metadata = hip_attn.get_scheduler_metadata(
        num_reqs=n,
        num_heads=attn.num_heads,
        num_kv_heads=attn.num_heads,
        head_dim=attn.head_dim,
        seq_lens=seq_lens,
        dtype=attn.k_cache.dtype,
        causal=False,
        isa=isa,
        block_size=block_size,
        group_start=group_start,
        group_order=group_order,
        max_group_size=max_group,
        active_groups=active,
        slot_descriptors=desc,
    )
    return [
        (
            layer.encoder_attn.k_cache,
            layer.encoder_attn.v_cache,
            block_table,
            seq_lens,
            metadata,
        )
        for layer in layers
    ]


def reshape_and_cache(key, value, k_cache, v_cache, slot_mapping, isa=None) -> None:
    """KV slot write into a paged pool (the runner's encoder path uses it directly)."""
    hip_attn.reshape_and_cache(key, value, k_cache, v_cache, slot_mapping, isa=isa)


@torch.library.custom_op("vflorence::self_attention", mutates_args={"k_cache", "v_cache"})
def decoder_self_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    """Write new K/V into the paged cache and run self-attention."""
    ctx = get_context()
    out = query.new_empty(query.shape)
    meta = ctx.self_metadata
    if meta is not None and meta.fuse_kv_write:
        # The runner built the slots from block-manager tables: one launch writes the
        # new K/V and attends (same cache contents and output as the two calls below).
        hip_attn.self_attention_with_kv_write(
            query,
            key,
            value,
            k_cache,
            v_cache,
            out,
            ctx.context_lens,
            ctx.slot_mapping,
            scale=scale,
            block_table=ctx.block_tables,
            scheduler_metadata=meta,
        )
        return out
    hip_attn.reshape_and_cache(key, value, k_cache, v_cache, ctx.slot_mapping, isa=ctx.isa)
    # One query per sequence, the newest token; the cache holds nothing after it, so
    # attending to the whole context is the causal result.
    hip_attn.attention_with_kv_cache(
        query,
        k_cache,
        v_cache,
        out,
        ctx.query_start_loc,
        ctx.context_lens,
        scale=scale,
        causal=False,
        block_table=ctx.block_tables,
        scheduler_metadata=ctx.self_metadata,
    )
    return out


@decoder_self_attention.register_fake
def _(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    scale: float,
) -> torch.Tensor:
    # The op returns a contiguous tensor (for the reference's strided q views,
    # empty_like gives the same layout).
    return query.new_empty(query.shape)


@torch.library.custom_op("vflorence::cross_attention", mutates_args={})
def decoder_cross_attention(
    query: torch.Tensor,
    layer_idx: int,
    scale: float,
) -> torch.Tensor:
    """Run cross-attention over the staged encoder K/V for decoder layer ``layer_idx``."""
    ctx = get_context()
    k_cache, v_cache, block_table, seq_lens, metadata = ctx.cross_staged[layer_idx]
    out = query.new_empty(query.shape)
    hip_attn.attention_with_kv_cache(
        query,
        k_cache,
        v_cache,
        out,
        ctx.query_start_loc,
        seq_lens,
        scale=scale,
        causal=False,
        block_table=block_table,
        scheduler_metadata=metadata,
    )
    return out


@decoder_cross_attention.register_fake
def _(query: torch.Tensor, layer_idx: int, scale: float) -> torch.Tensor:
    return query.new_empty(query.shape)
