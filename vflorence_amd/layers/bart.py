"""BART encoder-decoder whose decoder attention runs through the gfx950 paged ops.

The callers of the path (vflorence/models/bart.py:93-146): the decoder's self-attention
projects a fused q|k|v, views each third as ``[tokens, heads, head_dim]`` (strided
views, token stride 3 * d_model) and hands them to ``vflorence::self_attention``, which
writes k/v into this layer's paged pool and attends over the sequence's context; the
cross-attention projects q only and calls ``vflorence::cross_attention``, which reads
the encoder K/V that ``ModelRunner._encode`` paged once per request.  ``scaling`` is
``head_dim ** -0.5`` (:52).

Module and parameter names follow the transformers BART checkpoint layout
(``model.encoder.layers.N.self_attn...``, ``lm_head``, ``final_logits_bias``) so a
checkpoint's state dict loads after its q/k/v projections are concatenated
(``fuse_projections``).  The encoder runs dense attention with torch's SDPA on the
GPU: it is outside the decode path.  One decode step is ``forward(input_ids,
positions)`` over one token per running sequence.
"""

from __future__ import annotations

import math
from typing import NamedTuple

import torch
import torch.nn.functional as F
from torch import nn

from ..decoder_ops import LINEAR_MAX_IN, LINEAR_MAX_OUT, LINEAR_MAX_ROWS
from .attention import decoder_cross_attention, decoder_self_attention


def _residual_norm(h: torch.Tensor, y: torch.Tensor, norm: nn.LayerNorm) -> torch.Tensor:
    """``norm(h + y)``: one fused kernel on the GPU (vflorence_amd::add_layer_norm);
    torch's ops for host tensors (the encoder-only checks on the CPU)."""
    if h.is_cuda:
        from ..decoder_ops import add_layer_norm

        return add_layer_norm(y, h, norm.weight, norm.bias, norm.eps)
    return norm(h + y)


class PreNorm(NamedTuple):
    """A post-LN sublayer's output h' = LN(v) before its LayerNorm is applied: the
    pre-norm sum ``v`` ``[rows, d]``, its per-row, per-32-feature (mean, sum of squared
    deviations) ``stats`` ``[rows, d / 32, 2]`` and the LayerNorm's parameters.  The
    projections that read h' finish the normalization in their epilogue (their weights
    fold gamma and beta) and the next sublayer's output projection normalizes it as its
    residual, so no separate LayerNorm launch runs between the decoder's sublayers."""
    v: torch.Tensor
    stats: torch.Tensor
    gamma: torch.Tensor
    beta: torch.Tensor
    eps: float


def apply_pre_norm(h: "PreNorm | torch.Tensor") -> torch.Tensor:
    """The normalized tensor of a PreNorm (a plain tensor is returned as is)."""
    if isinstance(h, PreNorm):
        from ..decoder_ops import layer_norm_apply

        return layer_norm_apply(h.v, h.stats, h.gamma, h.beta, h.eps)
    return h


class DecodeLinear(nn.Linear):
    """nn.Linear whose decode-step calls -- at most 512 rows on the GPU times a 16-bit
    weight of up to 3072 outputs and 4096 inputs -- run on the split-K kernel
    (vflorence_amd::linear) with a copy of the weight re-laid out for it; other shapes,
    fp32 and host tensors go through F.linear (hipBLASLt on the GPU).

    The packed copy is made by ``repack`` (``load_model`` calls it after loading the
    weights) and rewritten in place, so HIP graphs captured over it stay valid.  An
    eager call also repacks when the weight's version counter moved (an in-place update
    of an ordinary tensor).  Inference tensors have no version counter: after updating
    such a weight in place call ``repack`` (``ModelRunner.repack_weights`` does it for
    the whole decoder), as also after any update that captured graphs must see."""

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        self._packed = None
        self._packed_key = None
        # The LayerNorm whose output this projection reads, when that output arrives as a
        # PreNorm (held in a tuple: a reference, not a submodule), and the operands with
        # it folded in (fold_layer_norm), refreshed by repack.
        self._in_norm = ()
        self._folded = None
        self._folded_key = None

    def set_input_norm(self, norm: nn.LayerNorm | None) -> None:
        """Declare the LayerNorm whose output this projection reads (None: its input is
        a plain tensor), so that it can take that input as a PreNorm."""
        self._in_norm = () if norm is None else (norm,)
        self._folded = None
        self._folded_key = None

    def _weight_key(self):
        w = self.weight
        version = None if w.is_inference() else w._version
        return (w.data_ptr(), version, w.dtype, tuple(w.shape))

    def repack(self) -> None:
        """Re-lay out the current weight into the packed copy (in place when one of the
        right size exists)."""
        from .. import decoder_ops

        w = self.weight
        if not (w.is_cuda and w.dtype in (torch.bfloat16, torch.float16)
                and decoder_ops.linear_fits(1, w, max_in=None, max_out=None)):
            self._packed = None
            self._packed_key = self._weight_key()
            self._refold()
            return
        out = self._packed
        if out is not None and (out.dtype != w.dtype or out.device != w.device
                                or out.numel() != decoder_ops.packed_elems(*w.shape)):
            out = None
        with torch.no_grad():
            self._packed = decoder_ops.pack_linear_weight(w.detach(), out=out)
        self._packed_key = self._weight_key()
        self._refold()

    def _fold_key(self):
        norm = self._in_norm[0]
        return (self._weight_key(),) + tuple(
            (t.data_ptr(), None if t.is_inference() else t._version)
            for t in (norm.weight, norm.bias) + (() if self.bias is None else (self.bias,)))

    def _refold(self) -> None:
        """Fold the input LayerNorm into a copy of the packed weight and the bias (in
        place when a copy of the right size exists)."""
        if not self._in_norm or self._packed is None:
            self._folded = None
            self._folded_key = None
            return
        from .. import decoder_ops

        norm = self._in_norm[0]
        out = self._folded
        if out is not None and out[0].numel() != self._packed.numel():
            out = None
        self._folded = decoder_ops.fold_layer_norm(self.weight.detach(), None if self.bias is None
                                                   else self.bias.detach(), norm.weight.detach(),
                                                   norm.bias.detach(), out=out)
        self._folded_key = self._fold_key()

    def folded_operands(self, rows: int, max_in: int | None = LINEAR_MAX_IN,
                        max_out: int | None = LINEAR_MAX_OUT):
        """(packed W', u, b') for a PreNorm input of ``rows`` rows, or None when this
        projection has no input LayerNorm or the kernel does not serve the call."""
        if not self._in_norm or self.kernel_weight(rows, max_in, max_out) is None:
            return None
        if not torch.compiler.is_compiling() and (self._folded_key is None
                                                  or self._fold_key() != self._folded_key):
            self._refold()
        return self._folded

    def packed_weight(self) -> torch.Tensor | None:
        """The weight in the kernel's packed layout (None when the kernel cannot take
        this weight).  Under torch.compile the copy made at load time is used as is
        (version counters are not traced; ``repack`` after an update)."""
        if torch.compiler.is_compiling():
            return self._packed
        if self._packed_key is None or self._weight_key() != self._packed_key:
            self.repack()
        return self._packed

    def kernel_weight(self, rows: int, max_in: int | None = LINEAR_MAX_IN,
                      max_out: int | None = LINEAR_MAX_OUT) -> torch.Tensor | None:
        """The packed weight when the split-K kernel serves ``rows`` rows of this
        projection (in / out features within ``max_in`` / ``max_out``), else None."""
        packed = self.packed_weight()
        if (packed is None or not 0 < rows <= LINEAR_MAX_ROWS
                or (max_in is not None and self.in_features > max_in)
                or (max_out is not None and self.out_features > max_out)):
            return None
        return packed

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.is_cuda and x.dtype == self.weight.dtype:
            packed = self.kernel_weight(x.numel() // x.shape[-1])
            if packed is not None:
                from .. import decoder_ops

                return decoder_ops.linear(x, packed, self.bias, self.out_features)
        return F.linear(x, self.weight, self.bias)

    def project(self, h: "PreNorm | torch.Tensor", flags: int = 0,
                max_out: int | None = LINEAR_MAX_OUT) -> torch.Tensor:
        """This projection of h, a plain tensor or a PreNorm of this projection's input
        LayerNorm (the deferred path; the caller has checked ``folded_operands``)."""
        from .. import decoder_ops

        if isinstance(h, PreNorm):
            packed, u, fb = self.folded_operands(h.v.shape[0], max_out=max_out)
            return decoder_ops.linear_norm(h.v, h.stats, h.eps, packed, u, fb,
                                           self.out_features, flags)
        packed = self.kernel_weight(h.shape[0], max_out=max_out)
        return decoder_ops.linear(h, packed, self.bias, self.out_features, flags=flags)

    def project_residual(self, x: torch.Tensor, residual: "PreNorm | torch.Tensor",
                         norm: nn.LayerNorm, rows: int = -1, flags: int = 0,
                         max_in: int | None = LINEAR_MAX_IN) -> PreNorm:
        """``norm(residual + self(x))`` as a PreNorm (post-LN sublayer output)."""
        from .. import decoder_ops

        n = rows if flags & decoder_ops.LINEAR_X_PACKED else x.shape[0]
        packed = self.kernel_weight(n, max_in=max_in)
        if isinstance(residual, PreNorm):
            v, st = decoder_ops.linear_residual(x, packed, self.bias, residual.v, residual.stats,
                                                residual.gamma, residual.beta, residual.eps,
                                                self.out_features, rows, flags)
        else:
            v, st = decoder_ops.linear_residual(x, packed, self.bias, residual, None, None, None,
                                                0.0, self.out_features, rows, flags)
        return PreNorm(v, st, norm.weight, norm.bias, norm.eps)


def _activation(name: str):
    from transformers.activations import ACT2FN

    return ACT2FN[name]


class BartLearnedPositionalEmbedding(nn.Embedding):
    """Learned positions with BART's offset of 2 (read through a view of the table that
    starts at the offset: no add kernel per step)."""

    OFFSET = 2

    def __init__(self, num_embeddings: int, embedding_dim: int):
        super().__init__(num_embeddings + self.OFFSET, embedding_dim)

    def forward(self, positions: torch.Tensor) -> torch.Tensor:
        return F.embedding(positions, self.weight[self.OFFSET:])


class BartScaledWordEmbedding(nn.Embedding):
    def __init__(self, num_embeddings, embedding_dim, padding_idx, embed_scale=1.0):
        super().__init__(num_embeddings, embedding_dim, padding_idx)
        self.embed_scale = embed_scale

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        out = super().forward(ids)
        return out if self.embed_scale == 1.0 else out * self.embed_scale


class _Heads(nn.Module):
    def __init__(self, embed_dim: int, num_heads: int):
        super().__init__()
        if embed_dim % num_heads:
            raise ValueError("embed_dim must be divisible by num_heads")
        self.embed_dim, self.num_heads = embed_dim, num_heads
        self.head_dim = embed_dim // num_heads
        self.scaling = self.head_dim**-0.5


class BartEncoderSelfAttention(_Heads):
    fused_projections = {"qkv_proj": ("q_proj", "k_proj", "v_proj")}

    def __init__(self, embed_dim: int, num_heads: int):
        super().__init__(embed_dim, num_heads)
        self.qkv_proj = nn.Linear(embed_dim, 3 * embed_dim)
        self.out_proj = nn.Linear(embed_dim, embed_dim)

    def attention(self, x: torch.Tensor, segments=None) -> torch.Tensor:
        """Attention output before ``out_proj``.  ``x``: [B, S, d] equal-length prompts,
        or with ``segments`` the [T, d] tokens of prompts stored back to back, where each
        ``(start, count, length)`` names ``count`` prompts of ``length`` tokens from token
        ``start`` on: the projection runs over all T tokens at once and attention per run
        of equal-length prompts."""
        if segments is None:
            b, s, _ = x.shape
            q, k, v = (t.view(b, s, self.num_heads, self.head_dim).transpose(1, 2)
                       for t in self.qkv_proj(x).chunk(3, dim=-1))
            out = F.scaled_dot_product_attention(q, k, v, scale=self.scaling)
            return out.transpose(1, 2).reshape(b, s, self.embed_dim)
        out = x.new_empty(x.shape[0], self.embed_dim)
        self.attend(self.qkv_proj(x), segments, out)
        return out

    def attend(self, qkv: torch.Tensor, segments, out: torch.Tensor) -> None:
        """Attention of each run of equal-length prompts over the packed projections
        ``qkv`` [>= T, 3 d], written to rows ``start .. start + count * length`` of
        ``out``; other rows are left as they are."""
        for start, count, length in segments:
            end = start + count * length
            q, k, v = (t.view(count, length, self.num_heads, self.head_dim).transpose(1, 2)
                       for t in qkv[start:end].chunk(3, dim=-1))
            o = F.scaled_dot_product_attention(q, k, v, scale=self.scaling)
            out[start:end].view(count, length, self.num_heads, self.head_dim).copy_(
                o.transpose(1, 2))

    def forward(self, x: torch.Tensor, segments=None) -> torch.Tensor:
        return self.out_proj(self.attention(x, segments))


class BartDecoderSelfAttention(_Heads):
    """One new token per running sequence; K/V go to the paged pool ``k_cache``/``v_cache``
    that the runner attaches (never reallocated)."""

    fused_projections = {"qkv_proj": ("q_proj", "k_proj", "v_proj")}

    def __init__(self, embed_dim: int, num_heads: int):
        super().__init__(embed_dim, num_heads)
        self.qkv_proj = DecodeLinear(embed_dim, 3 * embed_dim)
        self.out_proj = DecodeLinear(embed_dim, embed_dim)
        self.k_cache = self.v_cache = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = x.shape[0]
        return self.out_proj(self._attend(self.qkv_proj(x), n))

    def _attend(self, qkv: torch.Tensor, n: int) -> torch.Tensor:
        q, k, v = (t.view(n, self.num_heads, self.head_dim) for t in qkv.chunk(3, dim=-1))
        out = decoder_self_attention(q, k, v, self.k_cache, self.v_cache, self.scaling)
        return out.view(n, self.embed_dim)

    def attend(self, h: "PreNorm | torch.Tensor") -> torch.Tensor:
        """The attention output ``[n, d]`` before ``out_proj``, for the deferred path."""
        n = (h.v if isinstance(h, PreNorm) else h).shape[0]
        return self._attend(self.qkv_proj.project(h), n)


class BartDecoderCrossAttention(_Heads):
    """Queries only; the encoder K/V were paged by the runner (``kv_proj`` is used there)."""

    fused_projections = {"kv_proj": ("k_proj", "v_proj")}

    def __init__(self, embed_dim: int, num_heads: int, layer_idx: int):
        super().__init__(embed_dim, num_heads)
        self.q_proj = DecodeLinear(embed_dim, embed_dim)
        self.kv_proj = nn.Linear(embed_dim, 2 * embed_dim)
        self.out_proj = DecodeLinear(embed_dim, embed_dim)
        self.layer_idx = layer_idx
        self.k_cache = self.v_cache = None

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.out_proj(self._attend(self.q_proj(x)))

    def _attend(self, q: torch.Tensor) -> torch.Tensor:
        n = q.shape[0]
        out = decoder_cross_attention(q.view(n, self.num_heads, self.head_dim), self.layer_idx,
                                      self.scaling)
        return out.view(n, self.embed_dim)

    def attend(self, h: "PreNorm | torch.Tensor") -> torch.Tensor:
        """The attention output ``[n, d]`` before ``out_proj``, for the deferred path."""
        return self._attend(self.q_proj.project(h))


class BartEncoderLayer(nn.Module):
    def __init__(self, config):
        super().__init__()
        d = config.d_model
        self.self_attn = BartEncoderSelfAttention(d, config.encoder_attention_heads)
        self.self_attn_layer_norm = nn.LayerNorm(d)
        self.activation_fn = _activation(config.activation_function)
        self.fc1 = nn.Linear(d, config.encoder_ffn_dim)
        self.fc2 = nn.Linear(config.encoder_ffn_dim, d)
        self.final_layer_norm = nn.LayerNorm(d)

    def forward(self, h: torch.Tensor, segments=None) -> torch.Tensor:
        return self.tail(h, self.self_attn.attention(h, segments))

    def tail(self, h: torch.Tensor, att: torch.Tensor) -> torch.Tensor:
        """The layer after its attention: output projection, residual + LayerNorm,
        feed-forward, residual + LayerNorm (row by row)."""
        h = _residual_norm(h, self.self_attn.out_proj(att), self.self_attn_layer_norm)
        return _residual_norm(h, self.fc2(self.activation_fn(self.fc1(h))), self.final_layer_norm)


class BartDecoderLayer(nn.Module):
    def __init__(self, config, layer_idx: int):
        super().__init__()
        d, heads = config.d_model, config.decoder_attention_heads
        self.self_attn = BartDecoderSelfAttention(d, heads)
        self.self_attn_layer_norm = nn.LayerNorm(d)
        self.encoder_attn = BartDecoderCrossAttention(d, heads, layer_idx)
        self.encoder_attn_layer_norm = nn.LayerNorm(d)
        self.activation_fn = _activation(config.activation_function)
        # the fused feed-forward path computes the exact GELU (transformers' "gelu")
        self._exact_gelu = config.activation_function == "gelu"
        self.fc1 = DecodeLinear(d, config.decoder_ffn_dim)
        self.fc2 = DecodeLinear(config.decoder_ffn_dim, d)
        self.final_layer_norm = nn.LayerNorm(d)

    def _feed_forward(self, h: torch.Tensor) -> torch.Tensor:
        """fc2(gelu(fc1(h))) (vflorence/models/bart.py:192-201).  For a decode step's rows
        in bf16/fp16 on the GPU: two vfl_linear launches -- fc1 with the GELU in its
        epilogue writing the packed layout, fc2 reading it -- else the three torch ops."""
        if h.is_cuda and self._exact_gelu and h.dtype == self.fc1.weight.dtype:
            from .. import decoder_ops as ops

            rows = h.numel() // h.shape[-1]
            w1 = self.fc1.kernel_weight(rows, max_out=None)
            w2 = self.fc2.kernel_weight(rows, max_in=None)
            if w1 is not None and w2 is not None:
                mid = ops.linear(h, w1, self.fc1.bias, self.fc1.out_features,
                                 flags=ops.LINEAR_GELU | ops.LINEAR_Y_PACKED)
                out = ops.linear(mid, w2, self.fc2.bias, self.fc2.out_features, rows=rows,
                                 flags=ops.LINEAR_X_PACKED)
                return out.view(*h.shape[:-1], self.fc2.out_features)
        return self.fc2(self.activation_fn(self.fc1(h)))

    def forward(self, h: torch.Tensor) -> torch.Tensor:
        h = _residual_norm(h, self.self_attn(h), self.self_attn_layer_norm)
        h = _residual_norm(h, self.encoder_attn(h), self.encoder_attn_layer_norm)
        return _residual_norm(h, self._feed_forward(h), self.final_layer_norm)

    def deferred_ready(self, h: "PreNorm | torch.Tensor", rows: int) -> bool:
        """Whether this layer's decode step can run with deferred LayerNorms for an input
        h of ``rows`` rows: every projection on the kernels, the LayerNorm-reading ones
        with their folded weights, exact GELU, 16-bit, d a multiple of 32."""
        sa, ca = self.self_attn, self.encoder_attn
        if not self._exact_gelu or sa.embed_dim % 32:
            return False
        qkv = (sa.qkv_proj.folded_operands(rows) if isinstance(h, PreNorm)
               else sa.qkv_proj.kernel_weight(rows))
        return (qkv is not None and ca.q_proj.folded_operands(rows) is not None
                and self.fc1.folded_operands(rows, max_out=None) is not None
                and sa.out_proj.kernel_weight(rows) is not None
                and ca.out_proj.kernel_weight(rows) is not None
                and self.fc2.kernel_weight(rows, max_in=None) is not None)

    def forward_deferred(self, h: "PreNorm | torch.Tensor") -> PreNorm:
        """The layer on the decode step's kernels with each sublayer's LayerNorm deferred
        to the projections that read its output (``deferred_ready`` said yes): 6 launches
        of vfl_linear_* and the two attention ops, no LayerNorm launch.  Returns the
        final LayerNorm's input as a PreNorm."""
        from .. import decoder_ops as ops

        sa, ca = self.self_attn, self.encoder_attn
        rows = (h.v if isinstance(h, PreNorm) else h).shape[0]
        h1 = sa.out_proj.project_residual(sa.attend(h), h, self.self_attn_layer_norm)
        h2 = ca.out_proj.project_residual(ca.attend(h1), h1, self.encoder_attn_layer_norm)
        mid = self.fc1.project(h2, flags=ops.LINEAR_GELU | ops.LINEAR_Y_PACKED, max_out=None)
        return self.fc2.project_residual(mid, h2, self.final_layer_norm, rows=rows,
                                         flags=ops.LINEAR_X_PACKED, max_in=None)


def _embed_scale(config) -> float:
    return math.sqrt(config.d_model) if config.scale_embedding else 1.0


class BartEncoder(nn.Module):
    def __init__(self, config):
        super().__init__()
        d = config.d_model
        self.embed_tokens = BartScaledWordEmbedding(config.vocab_size, d, config.pad_token_id,
                                                    _embed_scale(config))
        self.embed_positions = BartLearnedPositionalEmbedding(config.max_position_embeddings, d)
        self.layers = nn.ModuleList(BartEncoderLayer(config) for _ in range(config.encoder_layers))
        self.layernorm_embedding = nn.LayerNorm(d)

    def embed(self, input_ids, positions):
        return self.layernorm_embedding(self.embed_tokens(input_ids) + self.embed_positions(positions))

    def forward(self, input_ids, positions, segments=None):
        h = self.embed(input_ids, positions)
        for layer in self.layers:
            h = layer(h, segments)
        return h


class BartDecoder(nn.Module):
    def __init__(self, config):
        super().__init__()
        d = config.d_model
        self.embed_tokens = BartScaledWordEmbedding(config.vocab_size, d, config.pad_token_id,
                                                    _embed_scale(config))
        self.embed_positions = BartLearnedPositionalEmbedding(config.max_position_embeddings, d)
        self.layers = nn.ModuleList(BartDecoderLayer(config, i)
                                    for i in range(config.decoder_layers))
        self.layernorm_embedding = nn.LayerNorm(d)
        # Decode steps on the GPU defer each sublayer's LayerNorm to the projections that
        # read its output (PreNorm); False runs the separate residual + LayerNorm kernel.
        self.deferred_norms = True
        # The LayerNorm each projection reads (for the deferred path): the first layer's
        # q|k|v reads the embedding LayerNorm's output as a plain tensor.
        for i, layer in enumerate(self.layers):
            if i > 0:
                layer.self_attn.qkv_proj.set_input_norm(self.layers[i - 1].final_layer_norm)
            layer.encoder_attn.q_proj.set_input_norm(layer.self_attn_layer_norm)
            layer.fc1.set_input_norm(layer.encoder_attn_layer_norm)

    def embed(self, input_ids, positions):
        """``layernorm_embedding(embed_tokens(ids) + embed_positions(positions))``
        (vflorence/models/bart.py:260-264): on the GPU one launch that looks up both rows
        and normalizes their sum (vflorence_amd::embed_layer_norm), the same arithmetic as
        the lookups followed by the residual + LayerNorm kernel."""
        tok, pos, ln = self.embed_tokens, self.embed_positions, self.layernorm_embedding
        d = tok.weight.shape[1]
        if (input_ids.is_cuda and input_ids.dim() == 1 and input_ids.dtype == torch.int64
                and positions.dtype == torch.int64 and d % 4 == 0 and d <= 4096
                and tok.weight.dtype == pos.weight.dtype == ln.weight.dtype):
            from ..decoder_ops import embed_layer_norm

            return embed_layer_norm(input_ids, positions, tok.weight, float(tok.embed_scale),
                                    pos.weight, pos.OFFSET, ln.weight, ln.bias, ln.eps)
        return _residual_norm(tok(input_ids), pos(positions), ln)

    def forward(self, input_ids, positions):
        h = self.embed(input_ids, positions)
        rows = h.shape[0]
        if (h.is_cuda and h.dim() == 2 and h.dtype in (torch.bfloat16, torch.float16)
                and self.deferred_norms):
            for layer in self.layers:
                if not layer.deferred_ready(h, rows):
                    h = layer(apply_pre_norm(h))
                else:
                    h = layer.forward_deferred(h)
            return apply_pre_norm(h)
        for layer in self.layers:
            h = layer(h)
        return h


class BartModel(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.shared = BartScaledWordEmbedding(config.vocab_size, config.d_model,
                                              config.pad_token_id, _embed_scale(config))
        self.encoder = BartEncoder(config)
        self.decoder = BartDecoder(config)
        if config.tie_word_embeddings:
            self.encoder.embed_tokens.weight = self.shared.weight
            self.decoder.embed_tokens.weight = self.shared.weight


# The LM head's GEMM runs on a copy of its weight and bias padded with zero rows to a
# multiple of this many outputs (16-bit weights on the GPU).  hipBLASLt at 256 rows x
# 1024 inputs (bf16): 50265 outputs 43.9-45.1 us, 50432 (197 x 256) 34.1-35.3 us;
# 51289 outputs 41.9-43.2 us, 51456 34.6 us.
LM_HEAD_MULTIPLE = 256


class BartForConditionalGeneration(nn.Module):
    def __init__(self, config):
        super().__init__()
        self.config = config
        self.model = BartModel(config)
        self.register_buffer("final_logits_bias", torch.zeros(1, config.vocab_size))
        self.lm_head = nn.Linear(config.d_model, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.shared.weight
        self._lm_padded = None  # (weight [Vp, d], bias [Vp]) or None
        self._lm_key = None

    @property
    def decoder_layers(self):
        return self.model.decoder.layers

    @torch.no_grad()
    def encode(self, encoder_token_ids: torch.Tensor) -> torch.Tensor:
        """Encoder hidden states [B, S, d_model] of equal-length prompts [B, S]."""
        b, s = encoder_token_ids.shape
        positions = torch.arange(s, device=encoder_token_ids.device).expand(b, s)
        return self.model.encoder(encoder_token_ids, positions)

    @torch.no_grad()
    def encode_packed(self, token_ids: torch.Tensor, positions: torch.Tensor,
                      segments) -> torch.Tensor:
        """Encoder hidden states [T, d_model] of prompts of any lengths stored back to back
        in ``token_ids`` / ``positions`` [T]; ``segments`` lists ``(start, count,
        length)`` runs of equal-length prompts covering the T tokens in order."""
        at = 0
        for start, count, length in segments:
            if start != at or count <= 0 or length <= 0:
                raise ValueError(f"segment ({start}, {count}, {length}) does not start at "
                                 f"token {at} or is empty")
            at += count * length
        if at != token_ids.shape[0] or positions.shape != token_ids.shape:
            raise ValueError(f"segments cover {at} tokens of {token_ids.shape[0]}")
        return self.model.encoder(token_ids, positions, segments)

    def _lm_head_key(self):
        w, b = self.lm_head.weight, self.final_logits_bias
        return tuple((t.data_ptr(), None if t.is_inference() else t._version, t.dtype,
                      tuple(t.shape)) for t in (w, b))

    def repack_lm_head(self) -> None:
        """Copy the LM head's weight and the final logits bias into the padded operands
        (in place when copies of the right size exist; None when the weight is not a
        16-bit GPU tensor or needs no padding)."""
        w = self.lm_head.weight
        vocab, d = w.shape
        padded = -(-vocab // LM_HEAD_MULTIPLE) * LM_HEAD_MULTIPLE
        self._lm_key = self._lm_head_key()
        if not (w.is_cuda and w.dtype in (torch.bfloat16, torch.float16)) or padded == vocab:
            self._lm_padded = None
            return
        ops = self._lm_padded
        if ops is None or ops[0].shape != (padded, d) or ops[0].dtype != w.dtype \
                or ops[0].device != w.device:
            ops = (torch.zeros(padded, d, dtype=w.dtype, device=w.device),
                   torch.zeros(padded, dtype=w.dtype, device=w.device))
        with torch.no_grad():
            ops[0][:vocab].copy_(w)
            ops[1][:vocab].copy_(self.final_logits_bias[0])
        self._lm_padded = ops

    def logits(self, h: torch.Tensor) -> torch.Tensor:
        """The LM head over decoder outputs ``h`` [N, d]: logits [N, vocab], the final
        logits bias added by the GEMM itself.  With padded operands the logits are the
        first ``vocab`` columns of the padded GEMM's output (a view whose rows are
        ``LM_HEAD_MULTIPLE``-aligned in memory).  An eager call re-copies the operands
        when the weight or bias version moved; under torch.compile and in captured
        graphs the copy made at load time is used (``repack_lm_head`` after an update)."""
        if not torch.compiler.is_compiling() and self._lm_key != self._lm_head_key():
            self.repack_lm_head()
        ops = self._lm_padded
        if ops is None:
            return F.linear(h, self.lm_head.weight, self.final_logits_bias[0])
        return F.linear(h, ops[0], ops[1])[:, : self.lm_head.weight.shape[0]]

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """One decode step: logits [N, vocab] for one token per running sequence."""
        return self.logits(self.model.decoder(input_ids, positions))


def fuse_projections(model: nn.Module, state_dict: dict) -> None:
    """Concatenate a checkpoint's separate projections (q/k/v_proj -> qkv_proj,
    k/v_proj -> kv_proj) along the output dimension, in place."""
    for prefix, module in model.named_modules():
        for target, sources in getattr(module, "fused_projections", {}).items():
            for suffix in ("weight", "bias"):
                names = [f"{prefix}.{s}.{suffix}" for s in sources]
                if all(n in state_dict for n in names):
                    state_dict[f"{prefix}.{target}.{suffix}"] = torch.cat(
                        [state_dict.pop(n) for n in names], dim=0)
