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
  order, block tables) is packed on the host into one pinned buffer at fixed offsets
  and sent with one asynchronous host->device copy; the Context holds views of the
  device copy (model_runner.py:273-341);
* the self-attention op receives a scheduler metadata that enables the fused KV write:
  the block manager's copy-on-write rule guarantees each row writes its last context
  position in a block no other row reads;
* encoder K/V are projected on the device and scattered into pages with one
  ``reshape_and_cache`` per layer (model_runner.py:208-259);
* logits rules and top-k run on the device; only the chosen ids (greedy) or each
  row's top-k (beam search) come back to the host.
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

logger = logging.getLogger(__name__)


class _StepBuffers:
    """Pinned host staging and its device twin for one step's metadata.

    int32 word layout for ``rows`` sequences and tables ``width`` blocks wide:
    six int64 vectors of ``rows`` (token ids, positions, slots, copy sources, copy
    destinations, lengths), then int32 context lengths, dispatch order, the row groups'
    starts (``rows + 1``) and the ``[rows, width]`` block tables.
    """

    I64 = ("input_ids", "positions", "slots", "copy_src", "copy_dst", "lengths")

    def __init__(self, rows: int, width: int, device):
        self.rows, self.width = rows, width
        words = 12 * rows + 3 * rows + 1 + rows * width
        self.host = torch.zeros(words, dtype=torch.int32, pin_memory=True)
        self.dev = torch.zeros(words, dtype=torch.int32, device=device)
        self.copied = torch.cuda.Event()
        self.copied.record()
        self.h = self._views(self.host)
        self.d = self._views(self.dev)
        self.np = {k: v.numpy() for k, v in self.h.items()}

    def _views(self, buf):
        r, w = self.rows, self.width
        out = {name: buf[2 * r * i: 2 * r * (i + 1)].view(torch.int64)
               for i, name in enumerate(self.I64)}
        out["context_lens"] = buf[12 * r: 13 * r]
        out["order"] = buf[13 * r: 14 * r]
        out["group_start"] = buf[14 * r: 15 * r + 1]
        out["tables"] = buf[15 * r + 1: 15 * r + 1 + r * w].view(r, w)
        return out

    def upload(self) -> None:
        self.dev.copy_(self.host, non_blocking=True)
        self.copied.record()


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


def _row_groups(seqs, max_group: int) -> list[int]:
    """Starts of the runs of rows that belong to one request (its beams, adjacent in the
    running list, vflorence/engine/scheduler.py:121-126), cut every ``max_group`` rows,
    followed by the row count."""
    starts = [0]
    for i in range(1, len(seqs)):
        if seqs[i].request_id != seqs[i - 1].request_id or i - starts[-1] >= max_group:
            starts.append(i)
    starts.append(len(seqs))
    return starts


def _merge_equal_beam_groups(seqs, scores, ids, keep: int):
    """The per-request candidate merge, vectorised for the usual beam-search batch: each
    request's rows adjacent and every request with the same number of rows.  Returns
    None for any other batch (the general merge handles it).

    Equals sorting each request's candidates -- listed row by row, each row best first
    -- by score, stably, best first: a stable ascending sort of the negated scores.
    """
    n, k = scores.shape
    rids = [s.request_id for s in seqs]
    nb = 1
    while nb < n and rids[nb] == rids[0]:
        nb += 1
    if n % nb:
        return None
    heads = rids[::nb]
    groups = n // nb
    if len(set(heads)) != groups or not (
            np.array(rids).reshape(groups, nb) == np.array(heads)[:, None]).all():
        return None
    flat = scores.reshape(groups, nb * k)
    order = np.argsort(-flat, axis=1, kind="stable")[:, :keep]
    rows = order // k + (np.arange(groups) * nb)[:, None]
    toks = ids[rows, order % k].tolist()
    vals = np.take_along_axis(flat, order, axis=1).tolist()
    rows = rows.tolist()
    return {rid: [(seqs[r], t, v) for r, t, v in zip(rows[j], toks[j], vals[j])]
            for j, rid in enumerate(heads)}


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
        self._cross_buffers = attention.CrossStagingBuffers(
            config.max_num_seqs, math.ceil(config.max_encoder_len / self.block_size), self.device)
        # decode steps captured per batch size (rows), replayed while the shapes repeat
        self._graphs: dict[tuple[int, bool], tuple[torch.cuda.CUDAGraph, torch.Tensor]] = {}
        self._step_grouped = False
        self._buckets = row_buckets(config.max_num_seqs)
        self._self_metadata: dict[tuple[int, bool], hip_attn.SchedulerMetadata] = {}
        self._no_pages = torch.zeros(0, dtype=torch.int32)
        self._graph_pool = torch.cuda.graph_pool_handle() if config.cuda_graphs else None

    def repack_weights(self) -> None:
        """Make the decoder's packed projection weights follow the current weights, after
        an in-place weight update (the copies are rewritten in place, so captured decode
        steps stay valid)."""
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
        mb = 1024**2
        weights = sum(t.nbytes for t in (*self.model.parameters(), *self.model.buffers()))
        kv = sum(c.nbytes for c in self._self_caches)
        logger.info("Allocated in HBM: weights %.1f MB, self KV %.1f MB (%d blocks), cross KV "
                    "%.1f MB (%d blocks)", weights / mb, kv / mb, cfg.num_blocks,
                    2 * len(self.decoder_layers) * math.prod(cross) * self.model.lm_head.weight
                    .element_size() / mb, cfg.num_cross_blocks)

    def _copy_blocks(self, copies, src: torch.Tensor | None = None,
                     dst: torch.Tensor | None = None) -> None:
        """Copy-on-write of ``(src, dst)`` block pairs in every self-attention pool, one
        launch (model_runner.py:162-167)."""
        if not copies:
            return
        if src is None:
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
        """Encoder forward per group of equal prompt length, then page each layer's
        cross-attention K/V (model_runner.py:208-259)."""
        groups = defaultdict(list)
        for seq in seqs:
            if seq.pixel_values is not None:
                raise ValueError("pixel_values are only supported for Florence-2 checkpoints")
            groups[len(seq.encoder_token_ids)].append(seq)
        bs = self.block_size
        for enc_len, group in groups.items():
            ids = torch.tensor([s.encoder_token_ids for s in group], dtype=torch.long)
            hidden = self.model.encode(ids.to(self.device, non_blocking=True))
            per_seq = math.ceil(enc_len / bs)
            pages = torch.tensor(self._allocate_cross_pages(len(group) * per_seq),
                                 dtype=torch.int32).view(len(group), per_seq)
            token = torch.arange(enc_len)
            slots = (pages[:, token // bs].long() * bs + token % bs).flatten()
            for seq, seq_pages in zip(group, pages):
                self._cross_pages[seq.request_id] = (seq_pages, enc_len)
            slots = slots.to(self.device, non_blocking=True)
            rows = len(group) * enc_len
            for layer in self.decoder_layers:
                attn = layer.encoder_attn
                kv = attn.kv_proj(hidden).view(rows, 2 * attn.embed_dim)
                key, value = (t.view(rows, attn.num_heads, attn.head_dim)
                              for t in kv.chunk(2, dim=-1))
                attention.reshape_and_cache(key, value, attn.k_cache, attn.v_cache, slots,
                                            isa=self.isa)

    def clear_request(self, request_id: int) -> None:
        """Return a finished request's encoder pages; drop the staged cross state."""
        pages, _ = self._cross_pages.pop(request_id, ((), 0))
        self._cross_free.extend(int(p) for p in pages)
        self._cross_key = self._cross_staged = None

    def reset(self) -> None:
        """Return every encoder page to the pool (after an aborted batch)."""
        self._cross_pages.clear()
        self._cross_free = list(range(self.config.num_cross_blocks))
        self._cross_key = self._cross_staged = None

    # -- step metadata -----------------------------------------------------------------

    def _prepare(self, seqs, copies=()):
        """Stage the step's metadata in HBM, run the copy-on-write, publish the Context.

        Returns the device ``(input_ids, positions)`` of the one token fed per sequence,
        padded to the step's row bucket (``row_buckets``): padding rows feed token 0 at
        position 0 with a zero-length context and write no KV slot, so the rows of the
        real sequences come out as without padding and their logits are the first rows.
        """
        bs = self.block_size
        n = len(seqs)
        positions = np.fromiter((seq.num_cached_tokens for seq in seqs), np.int64, n)
        lengths = np.fromiter((len(seq.token_ids) for seq in seqs), np.int64, n)
        table_lens = np.fromiter((len(seq.block_table) for seq in seqs), np.int64, n)
        bad = np.flatnonzero(lengths - positions != 1)
        if bad.size:
            raise ValueError("each step must feed 1 token per sequence, got "
                             f"{lengths[bad[0]] - positions[bad[0]]}")
        if (positions // bs >= table_lens).any():
            raise ValueError("a sequence has no block for its write position "
                             "(BlockManager.ensure_capacity was not called)")
        # rows n .. padded-1 are padding: no token written, zero-length contexts
        padded = next((b for b in self._buckets if b >= n), n)
        buf = self._buffers
        width = int(table_lens.max())
        if padded > buf.rows or width > buf.width or len(copies) > buf.rows:
            buf = self._buffers = _StepBuffers(max(padded, len(copies), buf.rows),
                                               max(width, buf.width), self.device)
            self._graphs.clear()  # they read the old buffers
            self._self_metadata.clear()
        buf.copied.synchronize()  # the previous step's upload has left the staging
        h = buf.np
        w = buf.width
        tables = h["tables"]
        tables[:n] = [seq.block_table + [0] * (w - len(seq.block_table)) for seq in seqs]
        # the one token fed is the last of each sequence's token ids (at its position)
        h["input_ids"][:n] = [seq.token_ids[-1] for seq in seqs]
        h["positions"][:n] = positions
        h["lengths"][:n] = lengths
        # slot = block_table[pos // bs] * bs + pos % bs (model_runner.py:296-299)
        h["slots"][:n] = (tables[np.arange(n), positions // bs].astype(np.int64) * bs
                          + positions % bs)
        lens = positions + 1
        h["context_lens"][:n] = lens
        if padded > n:
            for name, value in (("input_ids", 0), ("positions", 0), ("slots", -1),
                                ("context_lens", 0), ("lengths", 1)):
                h[name][n:padded] = value
            h["tables"][n:padded] = 0
        # Beams of a request share their prefix blocks (copy-on-write forks): their
        # self-attention runs as one row group that reads each shared block once.  The
        # group list is padded with empty groups to n entries so that one launch shape
        # serves every batch of n rows.
        starts = _row_groups(seqs, hip_attn.MAX_GROUP_SIZE)
        grouped = len(starts) - 1 < n
        if grouped:  # padding rows are groups of one (zero output)
            starts += range(n + 1, padded + 1)
            num_groups = len(starts) - 1
            h["group_start"][: num_groups + 1] = starts
            h["group_start"][num_groups + 1: padded + 1] = padded
        else:  # one row per workgroup: longest context first
            h["order"][:padded] = hip_attn.longest_first(lens.tolist() + [0] * (padded - n))
        if copies:
            h["copy_src"][: len(copies)] = [s for s, _ in copies]
            h["copy_dst"][: len(copies)] = [d for _, d in copies]
        buf.upload()
        d = buf.d
        # copy-on-write first: this step writes into the now-private blocks
        self._copy_blocks(copies, d["copy_src"][: len(copies)], d["copy_dst"][: len(copies)])
        # the plan points at fixed views of the step buffers: one per (rows, grouped)
        self_metadata = self._self_metadata.get((padded, grouped))
        if self_metadata is None:
            if grouped:
                self_metadata = hip_attn.get_scheduler_metadata(
                    num_reqs=padded, num_heads=self.num_heads, num_kv_heads=self.num_heads,
                    head_dim=self.head_dim, dtype=self.dtype, block_size=bs,
                    group_start=d["group_start"][: padded + 1],
                    max_group_size=hip_attn.MAX_GROUP_SIZE, own_tables=True,
                    fuse_kv_write=True)
            else:
                self_metadata = hip_attn.get_scheduler_metadata(
                    num_reqs=padded, num_heads=self.num_heads, num_kv_heads=self.num_heads,
                    head_dim=self.head_dim, dtype=self.dtype, block_size=bs,
                    group_order=d["order"][:padded], fuse_kv_write=True)
            self._self_metadata[(padded, grouped)] = self_metadata
        self._step_grouped = grouped
        request_ids = tuple(seq.request_id for seq in seqs) + (None,) * (padded - n)
        if request_ids != self._cross_key:
            pages, enc_lens = zip(*(self._cross_pages[rid] for rid in request_ids[:n]))
            pages = pages + (self._no_pages,) * (padded - n)
            enc_lens = enc_lens + (0,) * (padded - n)
            self._cross_staged = attention.stage_cross(self.decoder_layers, pages, enc_lens, bs,
                                                       self.isa, buffers=self._cross_buffers)
            self._cross_key = request_ids
        set_context(
            context_lens=d["context_lens"][:padded],
            block_tables=d["tables"][:padded],
            slot_mapping=d["slots"][:padded],
            query_start_loc=self._query_start_loc[: padded + 1],
            self_metadata=self_metadata,
            isa=self.isa,
            cross_staged=self._cross_staged,
        )
        return d["input_ids"][:padded], d["positions"][:padded]

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

    def _sample(self, seqs, logits, lengths: torch.Tensor | None = None):
        """Greedy: one token id per sequence.  Beam search: ``{request_id: candidates}``
        (model_runner.py:355-381)."""
        sp = seqs[0].sampling_params
        processor = self._get_logits_processor(sp)
        device = logits.device
        if lengths is None:
            lengths = torch.tensor([len(s.token_ids) for s in seqs], dtype=torch.long,
                                   device=device)
        history = None
        if processor.needs_history:
            width = max(len(s.token_ids) for s in seqs)
            history = torch.tensor([[-1] * (width - len(s.token_ids)) + s.token_ids
                                    for s in seqs], dtype=torch.long).to(device)
        rules = processor.topk_rules() if logits.is_cuda else None
        keep = max(2, 1 + len(sp.eos_ids())) * sp.num_beams
        if rules is not None and (sp.num_beams == 1 or keep <= decoder_ops.MAX_K):
            # one kernel: log-softmax (beam search), the rules, the per-row top-k
            if sp.num_beams == 1:
                _, ids = decoder_ops.logprob_topk(logits, 1, log_softmax=False, lengths=lengths,
                                                  rules=rules)
                return ids[:, 0].tolist()
            top, ids = decoder_ops.logprob_topk(logits, min(keep, logits.shape[-1]),
                                                log_softmax=True, lengths=lengths, rules=rules)
            return self._merge_candidates(seqs, top, ids, keep)
        scores = logits.float()
        if sp.num_beams > 1:
            scores = torch.log_softmax(scores, dim=-1)
        scores = processor(history, scores, lengths)
        if sp.num_beams == 1:
            return scores.argmax(dim=-1).tolist()
        return self._beam_search(seqs, scores, sp)

    def _beam_search(self, seqs, scores, sampling_params) -> dict[int, list]:
        """Each request's best ``max(2, 1 + n_eos) * num_beams`` continuations as
        ``(parent, token_id, cum_logprob)``, best first (model_runner.py:383-410).

        Per-row top-k runs on the device; only ``[rows, k]`` values and ids come back,
        and the per-request merge keeps the reference's ordering (a stable sort of the
        candidates listed row by row).
        """
        keep = max(2, 1 + len(sampling_params.eos_ids())) * sampling_params.num_beams
        top_scores, top_ids = torch.topk(scores, min(keep, scores.shape[-1]), dim=-1)
        return ModelRunner._merge_candidates(seqs, top_scores, top_ids, keep)

    @staticmethod
    def _merge_candidates(seqs, top_scores, top_ids, keep: int) -> dict[int, list]:
        """Add each row's cumulative log-prob to its top-k and keep every request's best
        ``keep`` candidates over its rows, best first."""
        top_scores, top_ids = _to_host(top_scores.float(), top_ids)
        scores, ids = top_scores.numpy(), top_ids.numpy()
        # each row's cumulative log-prob cast to float32 and added in float32
        # (model_runner.py:394-396)
        scores += np.array([s.cum_logprob for s in seqs], dtype=np.float32)[:, None]
        fast = _merge_equal_beam_groups(seqs, scores, ids, keep)
        if fast is not None:
            return fast
        candidates = defaultdict(list)
        for seq, row_scores, row_ids in zip(seqs, scores.tolist(), ids.tolist()):
            candidates[seq.request_id].extend(zip([seq] * len(row_ids), row_ids, row_scores))
        for cands in candidates.values():
            cands.sort(key=lambda c: c[2], reverse=True)
            del cands[keep:]
        return dict(candidates)

    # -- step ----------------------------------------------------------------------------

    @torch.inference_mode()
    def run(self, seqs, copies=()):
        """Encode fresh sequences, run one decoder step, return ``_sample``'s result."""
        if not seqs:
            return []
        fresh = [seq for seq in seqs if seq.num_cached_tokens == 0]
        if fresh:
            self._encode(fresh)
        try:
            input_ids, positions = self._prepare(seqs, copies)
            logits = self._forward(input_ids, positions)
        finally:
            set_context()
        n = len(seqs)  # the rows past n are padding
        return self._sample(seqs, logits[:n], self._buffers.d["lengths"][:n])

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
            return self.model(input_ids, positions)
        n = input_ids.shape[0]
        key = (n, self._step_grouped)  # grouped steps launch another kernel
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
