"""Per-step execution on one GPU: KV pools, encoder paging, step metadata, sampling.

Counterpart of vflorence/engine/model_runner.py:22-442 with the same public surface
(``run``, ``clear_request``, ``reset``, ``allocate_kv_cache``, ``_prepare``,
``_encode``, ``_copy_blocks``, ``_sample``, ``_beam_search``) and bookkeeping (the
encoder page pool and its free list, the per-batch cross-attention memo), laid out for
the GPU:

* every pool lives in HBM, one zero-filled tensor per layer and per K/V
  (model_runner.py:62-77); a device table of the self-attention pools' addresses is
  made once for the batched copy-on-write launch;
* a step's metadata (token ids, positions, slots, copy pairs, lengths, dispatch
  order, block tables) is written by the engine's native host core straight into one
  pinned buffer at fixed offsets and sent with one asynchronous host->device copy; the
  Context holds views of the device copy (model_runner.py:273-341);
* the self-attention op receives a scheduler metadata that enables the fused KV write:
  the block manager's copy-on-write rule guarantees each row writes its last context
  position in a block no other row reads;
* encoder K/V are projected on the device and scattered into pages with one
  ``reshape_and_cache`` per layer (model_runner.py:208-259);
* logits rules and top-k run on the device; only the chosen ids (greedy) or each
  row's top-k (beam search) come back to the host, where the host core merges a
  request's candidates.
"""

from __future__ import annotations

import logging
import math
from collections import defaultdict

import numpy as np
import torch

from .. import decoder_ops, hip_attn
from ..config import Config
from ..layers import attention
from ..layers.logits_processor import LogitsProcessor
from ..sampling_params import SamplingParams
from ..utils.context import set_context
from ..utils.loader import load_model
from .encoder_graphs import EncoderGraphs, page_cross_kv
from .._lib import check, lib

logger = logging.getLogger(__name__)


class _StepBuffers:
    """Pinned host staging and its device twin for one step's metadata.

    int32 word layout for ``rows`` sequences and tables ``width`` blocks wide:
    seven int64 vectors of ``rows`` (token ids, positions, slots, copy sources, copy
    destinations, lengths, row request ids), then int32 context lengths, dispatch
    order, the row groups' starts (``rows + 1``) and the ``[rows, width]`` block tables;
    last, 16-byte aligned, the group plan of the beam groups (``rows`` slots).  A step
    uploads the fixed part and the plan's used slots only.
    """

    I64 = ("input_ids", "positions", "slots", "copy_src", "copy_dst", "lengths",
           "row_requests")

    def __init__(self, rows: int, width: int, device):
        self.rows, self.width = rows, width
        fixed = 2 * len(self.I64) * rows + 3 * rows + 1 + rows * width
        self.plan_offset = (fixed + 3) // 4 * 4
        self.plan_stride = hip_attn.group_plan_stride(hip_attn.MAX_GROUP_SIZE, width)
        words = self.plan_offset + 4 + rows * self.plan_stride
        self.host = torch.zeros(words, dtype=torch.int32, pin_memory=True)
        self.dev = torch.zeros(words, dtype=torch.int32, device=device)
        # an upload the stream may not have finished: the staging must not be rewritten
        # before a synchronization (every step ends with one, in its sampling)
        self.in_flight = False
        self.h = self._views(self.host)
        self.d = self._views(self.dev)
        self.np = {k: v.numpy() for k, v in self.h.items()}
        self.ptr = {k: v.data_ptr() for k, v in self.h.items()}  # host staging addresses
        self._row_views: dict[int, tuple] = {}
        self._upload_views: dict[int, tuple] = {}

    def row_views(self, padded: int) -> tuple:
        """Device views of the first ``padded`` rows: (context lengths, block tables,
        slots, token ids, positions), made once per row count (a tensor slice costs
        ~2.5 us of host time, on the step's critical path)."""
        v = self._row_views.get(padded)
        if v is None:
            d = self.d
            v = self._row_views[padded] = (d["context_lens"][:padded], d["tables"][:padded],
                                           d["slots"][:padded], d["input_ids"][:padded],
                                           d["positions"][:padded])
        return v

    def _views(self, buf):
        r, w = self.rows, self.width
        out = {name: buf[2 * r * i: 2 * r * (i + 1)].view(torch.int64)
               for i, name in enumerate(self.I64)}
        base = 2 * len(self.I64) * r
        out["context_lens"] = buf[base: base + r]
        out["order"] = buf[base + r: base + 2 * r]
        out["group_start"] = buf[base + 2 * r: base + 3 * r + 1]
        out["tables"] = buf[base + 3 * r + 1: base + 3 * r + 1 + r * w].view(r, w)
        out["plan"] = buf[self.plan_offset:]
        return out

    def build_plan(self, padded: int, num_blocks: int, block_size: int) -> int:
        """The beam groups' plan for this step's ``padded`` rows, from the packed tables,
        lengths and group starts (slots = groups in row order, then empty ones); returns
        the number of groups."""
        gs = self.np["group_start"]
        groups = int(np.searchsorted(gs[: padded + 1], padded))
        p = self.ptr
        check(lib.vfl_build_group_plan(
            p["tables"], self.width, self.width, p["context_lens"], padded, p["group_start"],
            None, groups, block_size, num_blocks, p["plan"], self.rows, self.plan_stride))
        self._plan_words = 4 + groups * self.plan_stride
        return groups

    def fold_copies(self, num_pairs: int, num_blocks: int) -> bool:
        """Fold the packed copy-on-write pairs into the plan just built (the fused
        self-attention launches then copy the blocks); False when they cannot be."""
        p = self.ptr
        rc = lib.vfl_fold_plan_copies(p["plan"], self.rows, self.plan_stride, p["copy_src"],
                                      p["copy_dst"], num_pairs, num_blocks)
        return rc == 0

    def upload(self, grouped: bool = False) -> None:
        words = self.plan_offset + (self._plan_words if grouped else 0)
        v = self._upload_views.get(words)
        if v is None:
            v = self._upload_views[words] = (self.dev[:words], self.host[:words])
        v[0].copy_(v[1], non_blocking=True)
        self.in_flight = True  # (a flag, not an event: recording one costs ~4 us)


_HOST_STAGING: dict[tuple, torch.Tensor] = {}


def _to_host(*tensors: torch.Tensor) -> list[torch.Tensor]:
    """Device tensors copied to host memory with one synchronisation (pinned staging
    kept per shape and dtype; callers use the result before the next call)."""
    out = []
    for t in tensors:
        key = (tuple(t.shape), t.dtype, t.is_cuda)
        o = _HOST_STAGING.get(key)
        if o is None:
            o = _HOST_STAGING[key] = torch.empty(t.shape, dtype=t.dtype, pin_memory=t.is_cuda)
        o.copy_(t, non_blocking=True)
        out.append(o)
    if any(t.is_cuda for t in tensors):
        torch.cuda.current_stream().synchronize()
    return out


def _pinned(shape: tuple, dtype: torch.dtype) -> torch.Tensor:
    """A pinned host tensor kept per shape and dtype, for a kernel to write its result
    into (callers use it before asking for the same shape again)."""
    key = ("out", tuple(shape), dtype)
    o = _HOST_STAGING.get(key)
    if o is None:
        o = _HOST_STAGING[key] = torch.empty(shape, dtype=dtype, pin_memory=True)
    return o


def launch_slots(padded: int, below: int, beams: int, max_group: int) -> int:
    """Row-group slots an attention launch over a bucket of ``padded`` rows needs when
    its real rows are whole requests of ``beams`` rows each (more than ``below`` rows:
    the next smaller bucket), cut into groups of at most ``max_group`` rows, and the
    padding rows form groups of ``max_group``: the most groups any such batch makes.
    A launch sized this way spends no workgroups on slots no group can reach (64
    requests x 4 beams: 64 slots instead of 256).  ``padded`` when no row count of the
    bucket is a multiple of ``beams``.  A step whose groups exceed it (a request runs a
    single row on its first step) launches one slot per row instead."""
    per_request = -(-beams // max_group)
    most = 0
    for n in range(below + 1, padded + 1):
        if n % beams == 0:
            most = max(most, n // beams * per_request + -(-(padded - n) // max_group))
    return most or padded


def request_runs(row_requests: np.ndarray, padded: int, max_group: int) -> list[int]:
    """Group starts of a step's rows for the cross-attention staging: each run of rows
    of one request (beams are adjacent, scheduler.py:121-126; they read the same encoder
    pages) cut every ``max_group`` rows, then the padding rows up to ``padded`` in
    groups of ``max_group`` -- what ``attention.beam_groups`` finds by comparing the
    rows' pages.  Returns ``[0, ..., padded]``."""
    n = len(row_requests)
    starts = []
    if n:
        cuts = np.flatnonzero(row_requests[1:] != row_requests[:-1]) + 1
        bounds = [0, *cuts.tolist(), n]
        for a, b in zip(bounds, bounds[1:]):
            starts.extend(range(a, b, max_group))
    starts.extend(range(n, padded, max_group))
    starts.append(padded)
    return starts


def row_buckets(max_rows: int) -> list[int]:
    """Row counts a decode step is padded to: 1, 2, 4, 8, then steps of 8 up to 64, of 16
    up to 128, of 32 beyond, and ``max_rows`` itself.  A HIP graph is captured once per
    bucket, so a batch that changes size every step (continuous batching) replays a
    handful of graphs instead of capturing one per size."""
    sizes, s = [1, 2, 4, 8], 16
    while s < max_rows:
        sizes.append(s)
        s += 8 if s < 64 else 16 if s < 128 else 32
    return [b for b in sizes if b < max_rows] + [max_rows]


class ModelRunner:
    def __init__(self, config: Config, state_dict: dict | None = None):
        self.config = config
        self.device = torch.device(config.device)
        self.model = load_model(config, state_dict)
        self.block_size = config.block_size
        self.dtype = config.dtype
        self.decoder_layers = list(self.model.decoder_layers)
        self.num_heads = self.decoder_layers[0].self_attn.num_heads
        self.head_dim = self.decoder_layers[0].self_attn.head_dim
        if self.head_dim not in attention.HEAD_DIMS:
            raise ValueError(f"no gfx950 kernel for head_dim={self.head_dim}; "
                             f"must be one of {sorted(attention.HEAD_DIMS)}")
        self.isa = hip_attn.get_isa(self.dtype, self.block_size, self.head_dim)
        self.vocab_size = self.model.lm_head.out_features
        self._cross_pages: dict[int, tuple[torch.Tensor, int]] = {}
        self._cross_np: dict[int, np.ndarray] = {}  # the same pages as int32 numpy arrays
        self._cross_free = list(range(config.num_cross_blocks))
        self._cross_key = None
        self._cross_staged = None
        self._logits_processor: LogitsProcessor | None = None
        self._sampling_params: SamplingParams | None = None
        self.allocate_kv_cache()
        width = math.ceil(config.max_decoder_len / self.block_size) + 1
        self._buffers = _StepBuffers(config.max_num_seqs, width, self.device)
        self._query_start_loc = torch.arange(config.max_num_seqs + 1, dtype=torch.int32,
                                             device=self.device)
        self._qsl_views: dict[int, torch.Tensor] = {}  # its first padded + 1 entries
        self._cross_buffers = attention.CrossStagingBuffers(
            config.max_num_seqs, math.ceil(config.max_encoder_len / self.block_size), self.device)
        # decode steps captured per batch size (rows), replayed while the shapes repeat
        self._graphs: dict[tuple, tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self._step_grouped = False
        self._buckets = row_buckets(config.max_num_seqs)
        self._self_metadata: dict[tuple[int, bool, int], hip_attn.SchedulerMetadata] = {}
        self._slots: dict[tuple[int, int], int] = {}
        self._fold_copies = hip_attn.plan_copies_supported(self.dtype, self.head_dim,
                                                           self.block_size)
        self._step_slots = 0
        self.step_rows = self.step_pairs = 0
        self._no_pages = torch.zeros(0, dtype=torch.int32)
        self._no_pages_np = self._no_pages.numpy()
        self._graph_pool = torch.cuda.graph_pool_handle() if config.cuda_graphs else None
        # the packed encoder forward and K/V paging, captured per token bucket
        self._encoder_graphs = (EncoderGraphs(self.model, self.decoder_layers, self.isa)
                                if config.cuda_graphs else None)
        # the decoder step; compiled as the reference compiles it when asked
        # (vflorence/engine/model_runner.py:121-123)
        self.decode_fn = (torch.compile(self.model, dynamic=True) if config.compile
                          else self.model)

    def repack_weights(self) -> None:
        """Make the decoder's packed projection weights and the LM head's padded operands
        follow the current weights, after an in-place weight update (the copies are
        rewritten in place, so captured decode steps stay valid)."""
        from ..utils.loader import repack_decode_weights

        repack_decode_weights(self.model)

    # -- pools -------------------------------------------------------------------------

    def allocate_kv_cache(self) -> None:
        """Zero-filled pools in HBM, separate tensors per layer (model_runner.py:62-77)."""
        cfg = self.config
        shape = (cfg.num_blocks, self.num_heads, self.block_size, self.head_dim)
        cross = (cfg.num_cross_blocks, *shape[1:])
        for layer in self.decoder_layers:
            layer.self_attn.k_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
            layer.self_attn.v_cache = torch.zeros(shape, dtype=self.dtype, device=self.device)
            layer.encoder_attn.k_cache = torch.zeros(cross, dtype=self.dtype, device=self.device)
            layer.encoder_attn.v_cache = torch.zeros(cross, dtype=self.dtype, device=self.device)
        self._self_caches = [c for layer in self.decoder_layers
                             for c in (layer.self_attn.k_cache, layer.self_attn.v_cache)]
        self._cache_ptrs = hip_attn.cache_pointer_table(self._self_caches)
        self._copier = hip_attn.BlockCopier(self._self_caches)
        if hasattr(self, "_graphs"):  # a reallocation: what points at the old pools goes
            self._graphs.clear()
            self._cross_key = self._cross_staged = None
            if self._encoder_graphs is not None:
                self._encoder_graphs.clear()
        mb = 1024**2
        weights = sum(t.nbytes for t in (*self.model.parameters(), *self.model.buffers()))
        kv = sum(c.nbytes for c in self._self_caches)
        logger.info("Allocated in HBM: weights %.1f MB, self KV %.1f MB (%d blocks), cross KV "
                    "%.1f MB (%d blocks)", weights / mb, kv / mb, cfg.num_blocks,
                    2 * len(self.decoder_layers) * math.prod(cross) * self.model.lm_head.weight
                    .element_size() / mb, cfg.num_cross_blocks)

    def _copy_blocks(self, copies) -> None:
        """Copy-on-write of ``(src, dst)`` block pairs in every self-attention pool, one
        launch (model_runner.py:162-167)."""
        if not copies:
            return
        src = torch.tensor([s for s, _ in copies], dtype=torch.int64, device=self.device)
        dst = torch.tensor([d for _, d in copies], dtype=torch.int64, device=self.device)
        hip_attn.copy_blocks(self._self_caches, src, dst, self._cache_ptrs,
                             staged=hip_attn.copy_pairs_need_staging(copies))

    # -- encoder pages -----------------------------------------------------------------

    def _allocate_cross_pages(self, num_pages: int) -> list[int]:
        """Pages from the end of the encoder pool's free list (model_runner.py:169-177)."""
        if num_pages > len(self._cross_free):
            raise RuntimeError("encoder K/V pool is full; increase max_num_seqs or max_encoder_len")
        pages = self._cross_free[-num_pages:]
        del self._cross_free[-num_pages:]
        return pages

    def _encode(self, seqs) -> None:
        """Encode the step's admitted prompts and page each layer's cross-attention K/V
        (model_runner.py:208-259).  The reference runs one encoder forward per group of
        equal prompt length; here the groups' prompts are stored back to back and run as
        one forward (projections, LayerNorms and feed-forward over all of the step's
        tokens at once, attention per group), then one K/V scatter per layer covers every
        token; with HIP graphs on, that forward and the scatters replay from graphs
        captured per token bucket (``EncoderGraphs``), eagerly past the largest bucket.
        Pages are taken per group, in the reference's order."""
        groups = defaultdict(list)
        for seq in seqs:
            if seq.pixel_values is not None:
                raise ValueError("pixel_values are only supported for Florence-2 checkpoints")
            groups[len(seq.encoder_token_ids)].append(seq)
        if not groups:
            return
        bs = self.block_size
        ids, positions, slots, segments = [], [], [], []
        start = 0
        for enc_len, group in groups.items():
            per_seq = math.ceil(enc_len / bs)
            pages = torch.tensor(self._allocate_cross_pages(len(group) * per_seq),
                                 dtype=torch.int32).view(len(group), per_seq)
            for seq, seq_pages in zip(group, pages):
                self._cross_pages[seq.request_id] = (seq_pages, enc_len)
                self._cross_np[seq.request_id] = seq_pages.numpy()
            token = np.arange(enc_len)
            slots.append((pages.numpy()[:, token // bs].astype(np.int64) * bs
                          + token % bs).ravel())
            ids.extend(np.asarray(s.encoder_token_ids, dtype=np.int64) for s in group)
            positions.append(np.tile(token, len(group)))
            segments.append((start, len(group), enc_len))
            start += len(group) * enc_len
        ids, positions, slots = (np.concatenate(a) for a in (ids, positions, slots))
        if self._encoder_graphs is not None and self._encoder_graphs.run(ids, positions, slots,
                                                                         segments):
            return
        host = torch.from_numpy(np.concatenate([ids, positions, slots]))
        dev = host.to(self.device, non_blocking=True)
        ids_d, pos_d, slots_d = dev[:start], dev[start: 2 * start], dev[2 * start:]
        page_cross_kv(self.decoder_layers, self.model.encode_packed(ids_d, pos_d, segments),
                      slots_d, self.isa)

    def clear_request(self, request_id: int) -> None:
        """Return a finished request's encoder pages; drop the staged cross state."""
        pages, _ = self._cross_pages.pop(request_id, ((), 0))
        self._cross_np.pop(request_id, None)
        self._cross_free.extend(int(p) for p in pages)
        self._cross_key = self._cross_staged = None

    def reset(self) -> None:
        """Return every encoder page to the pool (after an aborted batch)."""
        self._cross_pages.clear()
        self._cross_np.clear()
        self._cross_free = list(range(self.config.num_cross_blocks))
        self._cross_key = self._cross_staged = None

    # -- step metadata -----------------------------------------------------------------

    def _prepare(self, batch):
        """Stage the step's metadata in HBM, run the copy-on-write, publish the Context.

        The host core writes the metadata of its scheduled rows into the pinned staging
        (model_runner.py:288-305 formulas: the fed token is each row's last, at position
        ``num_cached_tokens``; slot = table[pos // bs] * bs + pos % bs; context pos + 1).
        Returns the device ``(input_ids, positions)`` padded to the step's row bucket
        (``row_buckets``): padding rows feed token 0 at position 0 with a zero-length
        context and write no KV slot, so the real rows come out as without padding and
        their logits are the first rows.
        """
        core, n, num_pairs = batch.core, batch.num_rows, batch.num_pairs
        padded = next((b for b in self._buckets if b >= n), n)
        buf = self._buffers
        width = core.max_table_len()
        if padded > buf.rows or width > buf.width or num_pairs > buf.rows:
            buf = self._buffers = _StepBuffers(max(padded, num_pairs, buf.rows),
                                               max(width, buf.width), self.device)
            self._graphs.clear()  # they read the old buffers
            self._self_metadata.clear()
        if buf.in_flight:  # the previous upload must have left the staging
            torch.cuda.current_stream(self.device).synchronize()
            buf.in_flight = False
        h = buf.np
        # Beams of a request share their prefix blocks (copy-on-write forks): their
        # self-attention runs as row groups that read each shared block once; the group
        # list is padded with empty groups so one launch shape serves every n-row batch.
        grouped = core.pack(padded, buf.width, hip_attn.MAX_GROUP_SIZE, h)
        beams = batch.sampling_params.num_beams if batch.sampling_params else 1
        slots = self._launch_slots(padded, beams)
        folded = False
        if grouped:
            groups = buf.build_plan(padded, self.config.num_blocks, self.block_size)
            self_slots = slots if groups <= slots else padded
            # the copy-on-write rides in the self-attention launches: each layer's
            # launch copies the fork's block in its own pools (model_runner.py:284-286
            # order: the copy lands before the KV write, in the same launch)
            if num_pairs and self._fold_copies:
                folded = buf.fold_copies(num_pairs, self.config.num_blocks)
        else:
            self_slots = padded
        buf.upload(grouped)
        d = buf.d
        if num_pairs and not folded:  # copy-on-write first: this step writes into the
            # now-private blocks
            src, dst = h["copy_src"][:num_pairs], h["copy_dst"][:num_pairs]
            staged = not set(src.tolist()).isdisjoint(dst.tolist())
            self._copier(d["copy_src"][:num_pairs], d["copy_dst"][:num_pairs], staged=staged)
        # the plan points at fixed views of the step buffers: one per (rows, grouped,
        # group slots)
        bs = self.block_size
        self_metadata = self._self_metadata.get((padded, grouped, self_slots))
        if self_metadata is None:
            common = dict(num_reqs=padded, num_heads=self.num_heads, num_kv_heads=self.num_heads,
                          head_dim=self.head_dim, dtype=self.dtype, block_size=bs,
                          fuse_kv_write=True)
            if grouped:  # the groups' blocks come from the step's plan, self_slots slots
                plan = hip_attn.GroupPlan(d["plan"], buf.plan_stride, self_slots, buf.width)
                self_metadata = hip_attn.get_scheduler_metadata(
                    group_start=d["group_start"][: self_slots + 1],
                    max_group_size=hip_attn.MAX_GROUP_SIZE, own_tables=True,
                    group_plan=plan, **common)
            else:  # one row per workgroup, longest context first
                self_metadata = hip_attn.get_scheduler_metadata(
                    group_order=d["order"][:padded], **common)
            self._self_metadata[(padded, grouped, self_slots)] = self_metadata
        self._step_grouped = grouped
        self._step_slots = self_slots
        rows = h["row_requests"][:n]
        key = (padded, rows.tobytes())
        if key != self._cross_key:
            request_ids = rows.tolist()
            pages = [self._cross_np[rid] for rid in request_ids]
            pages += [self._no_pages_np] * (padded - n)
            enc_lens = [self._cross_pages[rid][1] for rid in request_ids] + [0] * (padded - n)
            self._cross_staged = attention.stage_cross(
                self.decoder_layers, pages, enc_lens, bs, self.isa, buffers=self._cross_buffers,
                slots=slots, group_starts=request_runs(rows, padded, hip_attn.MAX_GROUP_SIZE))
            self._cross_key = key
        context_lens, tables, slot_mapping, input_ids, positions = buf.row_views(padded)
        qsl = self._qsl_views.get(padded)
        if qsl is None:
            qsl = self._qsl_views[padded] = self._query_start_loc[: padded + 1]
        set_context(
            context_lens=context_lens,
            block_tables=tables,
            slot_mapping=slot_mapping,
            query_start_loc=qsl,
            self_metadata=self_metadata,
            isa=self.isa,
            cross_staged=self._cross_staged,
        )
        return input_ids, positions

    def _launch_slots(self, padded: int, beams: int) -> int:
        """Group slots of this bucket's attention launches at this beam width."""
        key = (padded, beams)
        slots = self._slots.get(key)
        if slots is None:
            i = self._buckets.index(padded) if padded in self._buckets else -1
            below = self._buckets[i - 1] if i > 0 else 0
            slots = self._slots[key] = launch_slots(padded, below, beams,
                                                    hip_attn.MAX_GROUP_SIZE)
        return slots

    # -- sampling ----------------------------------------------------------------------

    def _get_logits_processor(self, sampling_params: SamplingParams) -> LogitsProcessor:
        if sampling_params != self._sampling_params or self._logits_processor is None:
            # lengths count the decoder start token, as transformers does
            self._logits_processor = LogitsProcessor(
                sampling_params, vocab_size=self.vocab_size,
                max_length=1 + sampling_params.max_tokens,
                begin_index=1 + int(sampling_params.forced_bos_token_id is not None),
                device=self.device)
            self._sampling_params = sampling_params
        return self._logits_processor

    def _sample(self, batch, logits, lengths: torch.Tensor):
        """Greedy: each row's token id.  Beam search: each row's best
        ``max(2, 1 + n_eos) * num_beams`` processed log-probs and token ids, best first
        (model_runner.py:355-398); the host core merges a request's rows.  Host numpy
        arrays either way."""
        sp = batch.sampling_params
        processor = self._get_logits_processor(sp)
        history = None
        if processor.needs_history:
            history = torch.from_numpy(batch.core.history()).to(logits.device,
                                                                 non_blocking=True)
        rules = processor.topk_rules() if logits.is_cuda else None
        keep = max(2, 1 + len(sp.eos_ids())) * sp.num_beams
        if rules is not None and (sp.num_beams == 1 or keep <= decoder_ops.MAX_K):
            # one kernel: log-softmax (beam search), the rules, the per-row top-k, its
            # result stored by the kernel straight into pinned host memory (no copy
            # launches at the end of the step)
            k = 1 if sp.num_beams == 1 else min(keep, logits.shape[-1])
            rows = logits.shape[0]
            out = (_pinned((rows, k), torch.float32), _pinned((rows, k), torch.int64))
            top, ids = decoder_ops.logprob_topk(logits, k, log_softmax=sp.num_beams > 1,
                                                lengths=lengths, rules=rules, out=out)
            torch.cuda.current_stream().synchronize()
            if sp.num_beams == 1:
                return ids[:, 0].numpy()
            return top.numpy(), ids.numpy()
        scores = logits.float()
        if sp.num_beams > 1:
            scores = torch.log_softmax(scores, dim=-1)
        scores = processor(history, scores, lengths)
        if sp.num_beams == 1:
            return _to_host(scores.argmax(dim=-1))[0].numpy()
        return self._beam_search(scores, sp)

    def _beam_search(self, scores, sampling_params):
        """Each row's best ``max(2, 1 + n_eos) * num_beams`` continuations
        (model_runner.py:383-393) on the device: ([rows, k] scores, [rows, k] ids) on
        the host."""
        keep = max(2, 1 + len(sampling_params.eos_ids())) * sampling_params.num_beams
        top, ids = torch.topk(scores, min(keep, scores.shape[-1]), dim=-1)
        top, ids = _to_host(top, ids)
        return top.numpy(), ids.numpy()

    # -- step ----------------------------------------------------------------------------

    @torch.inference_mode()
    def run(self, batch):
        """Encode the step's newly admitted requests, run one decoder step over the
        scheduled rows, return ``_sample``'s result (None for an empty step)."""
        self.step_rows = batch.num_rows  # rows of the latest step (packed in _buffers)
        self.step_pairs = batch.num_pairs  # its copy-on-write pairs
        if batch.num_rows == 0:
            return None
        if batch.fresh:
            self._encode(batch.fresh)
        try:
            input_ids, positions = self._prepare(batch)
            logits = self._forward(input_ids, positions)
        finally:
            set_context()
        n = batch.num_rows  # the rows past n are padding
        out = self._sample(batch, logits[:n], self._buffers.d["lengths"][:n])
        self._buffers.in_flight = False  # sampling synchronized the stream
        return out

    def _forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """The decoder step, eager or replayed from a HIP graph of this batch size.

        Every tensor the step reads -- token ids, positions, the Context's lengths,
        tables and slots, the cross-attention staging -- lives at a fixed address for a
        given row count, and the launch shapes depend on the row count only, so one
        capture per row count serves every later step of that size.  The first step of
        a size runs eagerly (initialising libraries) before the capture; its KV write
        repeats in the replay with the same values.
        """
        if not self.config.cuda_graphs:
            return self.decode_fn(input_ids, positions)
        n = input_ids.shape[0]
        # grouped steps launch another kernel; the cross-attention's wave count follows
        # the batch's number of requests (one capture per count the batches use)
        cross_meta = self._cross_staged[0][4]
        cross_waves = cross_meta.plan(n, self._cross_buffers.max_pages).waves_per_workgroup
        key = (n, self._step_grouped, cross_waves, self._step_slots, cross_meta.num_groups)
        entry = self._graphs.get(key)
        if entry is None:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self.model(input_ids, positions)
            torch.cuda.current_stream().wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=self._graph_pool):
                logits = self.model(input_ids, positions)
            entry = self._graphs[key] = (graph, logits)
        graph, logits = entry
        graph.replay()
        return logits
