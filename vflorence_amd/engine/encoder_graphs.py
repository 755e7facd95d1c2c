"""HIP graphs of the packed encoder forward and the cross-attention K/V paging.

A step's admitted prompts run as one packed encoder forward (``ModelRunner._encode``,
the counterpart of vflorence/engine/model_runner.py:208-259).  Its token count changes
from step to step, and run eagerly each of its ~180 launches costs more host time than
GPU time (hipBLASLt chooses an algorithm for every new row count).  Here the row-wise
part of the forward -- embeddings, projections, LayerNorms and feed-forward, then the
K/V projections and paging of every decoder layer -- is captured per token bucket (the
step's tokens padded up to it): one graph before the first layer's attention, one
between each layer's attention and the next, the last ending with the paging.  The
attention of each run of equal-length prompts runs eagerly between them, over the real
tokens only.  Padding tokens are row-wise values that nothing reads: attention leaves
them out and their K/V slots are -1, which the slot write skips.
"""

from __future__ import annotations

import numpy as np
import torch

from ..layers import attention


def page_cross_kv(decoder_layers, hidden: torch.Tensor, slots: torch.Tensor, isa) -> None:
    """Each decoder layer's cross-attention K/V of encoder outputs ``hidden`` [T, d],
    written to the int64 ``slots`` [T] of its encoder pool (negative: skipped)
    (vflorence/engine/model_runner.py:236-259)."""
    rows = hidden.shape[0]
    for layer in decoder_layers:
        attn = layer.encoder_attn
        kv = attn.kv_proj(hidden)
        key, value = (t.view(rows, attn.num_heads, attn.head_dim) for t in kv.chunk(2, dim=-1))
        attention.reshape_and_cache(key, value, attn.k_cache, attn.v_cache, slots, isa=isa)


def token_bucket(tokens: int, max_tokens: int) -> int | None:
    """The padded token count a packed forward of ``tokens`` tokens runs at: a multiple
    of 256 up to 2048, of 512 beyond; None past ``max_tokens`` (run eagerly)."""
    if tokens <= 0 or tokens > max_tokens:
        return None
    step = 256 if tokens <= 2048 else 512
    return -(-tokens // step) * step


class _Bucket:
    """One bucket's static inputs, captured graphs and the tensors they hand on."""

    def __init__(self, tokens: int, d_model: int, dtype, device):
        self.tokens = tokens
        # token ids, positions, K/V slots: pinned staging and its device twin
        self.host = torch.zeros(3, tokens, dtype=torch.int64, pin_memory=True)
        self.np = self.host.numpy()
        self.dev = torch.zeros(3, tokens, dtype=torch.int64, device=device)
        self.dev[2].fill_(-1)
        self.copied = torch.cuda.Event()
        self.copied.record()
        # the current layer's q|k|v projections (written by a graph, read by the eager
        # attention) and the attention output (written by it, read by the next graph)
        self.qkv = torch.zeros(tokens, 3 * d_model, dtype=dtype, device=device)
        self.att = torch.zeros(tokens, d_model, dtype=dtype, device=device)
        self.graphs: list[torch.cuda.CUDAGraph] = []


class EncoderGraphs:
    """Captured packed encoder forwards of one model, per token bucket.  A bucket of T
    tokens holds its graphs' memory and two [T, 3 d] and [T, d] buffers for the process's
    life (at d = 1024, bf16, ~0.3 GB for the largest bucket; at most 20 buckets)."""

    def __init__(self, model, decoder_layers, isa, max_tokens: int = 8192):
        self.model = model
        self.encoder = model.model.encoder
        self.decoder_layers = decoder_layers
        self.isa = isa
        self.max_tokens = max_tokens
        self._buckets: dict[int, _Bucket] = {}

    def clear(self) -> None:
        """Drop every captured bucket (after the pools they page into were replaced)."""
        self._buckets.clear()

    def run(self, ids: np.ndarray, positions: np.ndarray, slots: np.ndarray, segments) -> bool:
        """Encode the packed prompts (int64 ``ids``, ``positions``, ``slots`` [T]) and
        page their K/V; False (nothing done) when T is past the largest bucket."""
        tokens = len(ids)
        size = token_bucket(tokens, self.max_tokens)
        if size is None:
            return False
        b = self._buckets.get(size)
        if b is None:
            b = self._buckets[size] = self._capture(size)
        b.copied.synchronize()  # the previous upload has left the staging
        b.np[0, :tokens] = ids
        b.np[1, :tokens] = positions
        b.np[2, :tokens] = slots
        b.np[:2, tokens:] = 0
        b.np[2, tokens:] = -1
        b.dev.copy_(b.host, non_blocking=True)
        b.copied.record()
        b.graphs[0].replay()
        for layer, graph in zip(self.encoder.layers, b.graphs[1:]):
            layer.self_attn.attend(b.qkv, segments, b.att)
            graph.replay()
        return True

    def _capture(self, size: int) -> _Bucket:
        layers = self.encoder.layers
        weight = layers[0].self_attn.qkv_proj.weight
        b = _Bucket(size, layers[0].self_attn.embed_dim, weight.dtype, weight.device)
        ids, pos, slots = b.dev[0], b.dev[1], b.dev[2]
        state = {}

        def project(layer, h):  # layer.self_attn.qkv_proj(h), into the bucket's buffer
            lin = layer.self_attn.qkv_proj
            if lin.bias is None:
                torch.mm(h, lin.weight.t(), out=b.qkv)
            else:
                torch.addmm(lin.bias, h, lin.weight.t(), out=b.qkv)

        def first():
            h = self.encoder.embed(ids, pos)
            project(layers[0], h)
            return h

        def middle(i):
            def piece():
                h = layers[i].tail(state["h"], b.att)
                project(layers[i + 1], h)
                return h
            return piece

        def last():
            h = layers[-1].tail(state["h"], b.att)
            # every slot is -1 until run() stages real ones
            page_cross_kv(self.decoder_layers, h, slots, self.isa)
            return h

        pieces = [first] + [middle(i) for i in range(len(layers) - 1)] + [last]
        pool = torch.cuda.graph_pool_handle()
        cur = torch.cuda.current_stream()
        for piece in pieces:
            side = torch.cuda.Stream()
            side.wait_stream(cur)
            with torch.cuda.stream(side):  # eager once: lazy initialisation outside capture
                piece()
            cur.wait_stream(side)
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, pool=pool):
                state["h"] = piece()
            b.graphs.append(graph)
        torch.cuda.synchronize()
        return b
