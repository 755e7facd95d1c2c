"""Seeded synthetic inputs for the decode attention path.

Shapes follow the BART-large / Florence-2 decoder (d_model 1024 -> 16 heads x 64, or
768 -> 12 x 64) with 16-token blocks.  Pools are filled on the device with a seeded
generator; callers that need the same bytes on the host copy them back.  Query, key
and value for the self-attention op are strided views of one fused [N, 3*E] tensor,
as the decoder's fused qkv projection produces them (vflorence/models/bart.py:108-112).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class SelfAttentionCase:
    """One decoder self-attention call: new token per sequence + paged context."""

    query: torch.Tensor  # [N, H, D] view, token stride 3E
    key: torch.Tensor  # [N, H, D] view
    value: torch.Tensor  # [N, H, D] view
    k_cache: torch.Tensor  # [NB, H, bs, D]
    v_cache: torch.Tensor
    context_lens: torch.Tensor  # int32 [N]
    block_tables: torch.Tensor  # int32 [N, max_blocks], 0-padded
    slot_mapping: torch.Tensor  # int64 [N]
    scale: float

    @property
    def num_seqs(self) -> int:
        return self.query.shape[0]


def fill_normal_(t: torch.Tensor, std: float, generator: torch.Generator) -> torch.Tensor:
    """Fill ``t`` with N(0, std^2) samples, generated in fp32 in chunks, then cast."""
    flat = t.view(-1)
    chunk = 1 << 26
    for start in range(0, flat.numel(), chunk):
        n = min(chunk, flat.numel() - start)
        tmp = torch.randn(n, generator=generator, device=t.device, dtype=torch.float32)
        flat[start : start + n].copy_(tmp.mul_(std))
    return t


def self_attention_case(
    num_seqs: int = 256,
    num_heads: int = 16,
    head_dim: int = 64,
    block_size: int = 16,
    pool_blocks: int = 20_000,
    min_ctx: int = 1,
    max_ctx: int = 1024,
    dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cuda",
    seed: int = 0,
    std: float = 1.0 / 8.0,
    context_lens: list[int] | None = None,
) -> SelfAttentionCase:
    """Op-level paged self-attention: ragged contexts over a random block permutation.

    Sequence s has ``L_s ~ U[min_ctx, max_ctx]`` tokens (the last being the new one)
    and takes the next ``ceil(L_s / bs)`` ids of a random permutation of the pool.
    The new token's slot is that of position ``L_s - 1``.
    """
    g = torch.Generator().manual_seed(seed)
    if context_lens is None:
        lens = torch.randint(min_ctx, max_ctx + 1, (num_seqs,), generator=g).tolist()
    else:
        lens = list(context_lens)
        num_seqs = len(lens)
    nblocks = [max(1, math.ceil(L / block_size)) for L in lens]
    if sum(nblocks) > pool_blocks:
        raise ValueError(f"pool of {pool_blocks} blocks cannot hold {sum(nblocks)}")
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    width = max(nblocks)
    tables, slots, pos = [], [], 0
    for L, nb in zip(lens, nblocks):
        row = perm[pos : pos + nb]
        pos += nb
        p = max(L, 1) - 1
        slots.append(row[p // block_size] * block_size + p % block_size)
        tables.append(row + [0] * (width - nb))
    dg = torch.Generator(device=device).manual_seed(seed + 1)
    E = num_heads * head_dim
    shape = (pool_blocks, num_heads, block_size, head_dim)
    k_cache = fill_normal_(torch.empty(shape, dtype=dtype, device=device), std, dg)
    v_cache = fill_normal_(torch.empty(shape, dtype=dtype, device=device), std, dg)
    qkv = fill_normal_(torch.empty((num_seqs, 3 * E), dtype=dtype, device=device), std, dg)
    q, k, v = (t.reshape(num_seqs, num_heads, head_dim) for t in qkv.chunk(3, dim=-1))
    return SelfAttentionCase(
        query=q,
        key=k,
        value=v,
        k_cache=k_cache,
        v_cache=v_cache,
        context_lens=torch.tensor(lens, dtype=torch.int32, device=device),
        block_tables=torch.tensor(tables, dtype=torch.int32, device=device),
        slot_mapping=torch.tensor(slots, dtype=torch.int64, device=device),
        scale=head_dim**-0.5,
    )


@dataclass
class CrossAttentionCase:
    """One decoder cross-attention call: beams of a request share encoder pages."""

    query: torch.Tensor  # [N, H, D] contiguous (N = requests * beams)
    k_cache: torch.Tensor  # [NCB, H, bs, D]
    v_cache: torch.Tensor
    pages: list[torch.Tensor]  # per row, int32 (beams repeat one tensor)
    enc_lens: list[int]  # per row
    scale: float


def cross_attention_case(
    num_requests: int = 64,
    beams: int = 4,
    num_heads: int = 16,
    head_dim: int = 64,
    block_size: int = 16,
    min_enc: int = 256,
    max_enc: int = 1024,
    dtype: torch.dtype = torch.bfloat16,
    device: str | torch.device = "cuda",
    seed: int = 0,
    std: float = 1.0,
    enc_lens: list[int] | None = None,
    pool_blocks: int | None = None,
) -> CrossAttentionCase:
    """Cross-attention over per-request encoder pages, taken from the end of a free list
    as ModelRunner._allocate_cross_pages does (vflorence/engine/model_runner.py:169-177)."""
    g = torch.Generator().manual_seed(seed)
    if enc_lens is None:
        lens = torch.randint(min_enc, max_enc + 1, (num_requests,), generator=g).tolist()
    else:
        lens = list(enc_lens)
        num_requests = len(lens)
    need = [math.ceil(L / block_size) for L in lens]
    if pool_blocks is None:
        pool_blocks = num_requests * math.ceil(max_enc / block_size)
    free = list(range(pool_blocks))
    pages, rows_lens = [], []
    for L, n in zip(lens, need):
        if n > len(free):
            raise ValueError("encoder pool too small")
        mine = free[-n:] if n else []
        del free[len(free) - n :]
        t = torch.tensor(mine, dtype=torch.int32)
        for _ in range(beams):
            pages.append(t)
            rows_lens.append(L)
    dg = torch.Generator(device=device).manual_seed(seed + 1)
    shape = (pool_blocks, num_heads, block_size, head_dim)
    k_cache = fill_normal_(torch.empty(shape, dtype=dtype, device=device), std, dg)
    v_cache = fill_normal_(torch.empty(shape, dtype=dtype, device=device), std, dg)
    n_rows = num_requests * beams
    query = fill_normal_(
        torch.empty((n_rows, num_heads, head_dim), dtype=dtype, device=device), std, dg
    )
    return CrossAttentionCase(
        query=query,
        k_cache=k_cache,
        v_cache=v_cache,
        pages=pages,
        enc_lens=rows_lens,
        scale=head_dim**-0.5,
    )


def self_attention_bytes(context_lens: list[int], num_heads: int, head_dim: int,
                         elem_bytes: int, block_size: int = 16) -> int:
    """Algorithmic HBM bytes of one self-attention call including the KV slot write:
    K/V of every context token once, q in + out, new k/v in + their cache write,
    block-table entries, lengths and slots."""
    N = len(context_lens)
    row = num_heads * head_dim * elem_bytes
    kv = sum(2 * L * row for L in context_lens)
    return (kv + 2 * N * row + 4 * N * row
            + sum(4 * math.ceil(L / block_size) for L in context_lens) + 12 * N)


def shared_self_attention_bytes(block_tables: list[list[int]], context_lens: list[int],
                                group_size: int, num_heads: int, head_dim: int,
                                elem_bytes: int, block_size: int = 16) -> int:
    """self_attention_bytes for rows taken in groups of ``group_size`` whose tables may
    list the same blocks (the beams of a request after copy-on-write forks): a block
    that several rows of a group list at one position is read once, for the most
    tokens any of those rows uses from it."""
    N = len(context_lens)
    row = num_heads * head_dim * elem_bytes
    tokens = 0
    for g0 in range(0, N, group_size):
        used: dict[tuple[int, int], int] = {}
        for r in range(g0, min(N, g0 + group_size)):
            L = context_lens[r]
            for i in range(math.ceil(L / block_size)):
                key = (i, block_tables[r][i])
                used[key] = max(used.get(key, 0), min(block_size, L - block_size * i))
        tokens += sum(used.values())
    return (2 * tokens * row + 2 * N * row + 4 * N * row
            + sum(4 * math.ceil(L / block_size) for L in context_lens) + 12 * N)


def cross_attention_bytes(enc_lens_per_group: list[int], num_rows: int, num_heads: int,
                          head_dim: int, elem_bytes: int, block_size: int = 16) -> int:
    """Algorithmic HBM bytes of one cross-attention call: each request's encoder K/V
    once (beams share it), q in + out per row, page-table entries and lengths."""
    row = num_heads * head_dim * elem_bytes
    kv = sum(2 * E * row for E in enc_lens_per_group)
    return (kv + 2 * num_rows * row
            + sum(4 * math.ceil(E / block_size) for E in enc_lens_per_group) + 4 * num_rows)


@dataclass
class DecodeStepPlan:
    """Host-side metadata of one decode step of the beam-search workload."""

    block_tables: list[list[int]]  # per row, unpadded
    context_lens: list[int]  # per row (position + 1)
    slot_mapping: list[int]  # per row
    copies: list[tuple[int, int]]  # copy-on-write pairs, copied before the KV write


def beam_decode_schedule(
    num_requests: int = 64,
    beams: int = 4,
    steps: int = 128,
    block_size: int = 16,
    num_blocks: int | None = None,
    cow_fraction: float = 0.10,
    seed: int = 0,
) -> list[DecodeStepPlan]:
    """Synthetic beam search driven through the real BlockManager.

    Every step each row feeds one token (ModelRunner._prepare, model_runner.py:288-300)
    after the scheduler's ensure_capacity pass (scheduler.py:124-134).  After the step,
    ``round(cow_fraction * blocks_in_use)`` beams (at most beams - 1 per request) are
    replaced by forks of a surviving sibling, as beam search re-ranks hypotheses
    (scheduler.py:193-199): the fork shares the parent's blocks, so the next step's
    write into the shared partial block produces one copy-on-write pair.  Beams of a
    request stay adjacent.
    """
    import random

    from .engine.block_manager import BlockManager
    from .engine.sequence import Sequence
    from .sampling_params import SamplingParams

    rng = random.Random(seed)
    n_rows = num_requests * beams
    if num_blocks is None:
        num_blocks = n_rows * math.ceil(steps / block_size)
    bm = BlockManager(num_blocks, block_size)
    params = SamplingParams(max_tokens=steps, num_beams=beams)
    rows = [Sequence(r, [0], [0], params) for r in range(num_requests) for _ in range(beams)]
    plans = []
    for t in range(steps):
        if bm.required_new_blocks(rows) > bm.num_free_blocks:
            raise RuntimeError("KV cache is full; increase num_blocks")
        copies = [c for seq in rows if (c := bm.ensure_capacity(seq)) is not None]
        tables, lens, slots = [], [], []
        for seq in rows:
            pos = seq.num_cached_tokens
            tables.append(list(seq.block_table))
            lens.append(pos + 1)
            slots.append(seq.block_table[pos // block_size] * block_size + pos % block_size)
        plans.append(DecodeStepPlan(tables, lens, slots, copies))
        for seq in rows:
            seq.num_cached_tokens += 1
            seq.token_ids.append(0)
        if t == steps - 1:
            break
        in_use = num_blocks - bm.num_free_blocks
        forks = min(round(cow_fraction * in_use), num_requests * (beams - 1))
        per_request = [0] * num_requests
        for _ in range(forks):
            candidates = [r for r in range(num_requests) if per_request[r] < beams - 1]
            if not candidates:
                break
            per_request[rng.choice(candidates)] += 1
        for r, m in enumerate(per_request):
            if m == 0:
                continue
            group = rows[r * beams : (r + 1) * beams]
            order = list(range(beams))
            rng.shuffle(order)
            victims, parents = order[:m], order[m:]
            for v in victims:
                parent = group[rng.choice(parents)]
                child = parent.fork(0, 0.0)
                child.num_cached_tokens = parent.num_cached_tokens
                bm.fork(parent, child)
                bm.deallocate(group[v])
                group[v] = child
            rows[r * beams : (r + 1) * beams] = group
    return plans
