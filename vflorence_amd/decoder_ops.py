"""torch wrappers of the decoder-step kernels around the attention path.

``add_layer_norm`` is the decoder layer's ``layer_norm(hidden + sublayer(hidden))``
(vflorence/models/bart.py:192-201) in one launch, registered as the custom op
``vflorence_amd::add_layer_norm`` so a compiled decoder keeps it whole.
``linear`` (custom op ``vflorence_amd::linear``) is nn.Linear for a decode step's rows
times a weight re-laid out once by ``pack_linear_weight`` (the decoder's q|k|v,
attention output and cross-attention query projections,
vflorence/models/bart.py:111,114,142,146); ``linear_fits`` says when it applies.
``logprob_topk`` is the device half of sampling (vflorence/engine/model_runner.py:355-398):
log-softmax, the history-free generation rules and the per-row top-k in one read of
the logits.  All run on the current stream; CPU tensors are rejected.
"""

from __future__ import annotations

import torch

from ._lib import check, lib
from .hip_attn import _dtype_code, _require_gpu, _stream

# largest k of logprob_topk (each lane keeps its k best in registers)
MAX_K = 16

# Where vfl_linear is used: measured on MI355X at 256 rows with the weight streamed
# from HBM (HIP-graph replays over more weight copies than the last-level cache holds),
# against hipBLASLt timed the same way: 5.3-5.6 against 10.5-10.7 us for 1024 x 1024,
# 9.4-10.0 against 11.8-11.9 us for the 3072 x 1024 q|k|v, 9.5-9.8 against 12.3 us for a
# 1024-wide, 4096-deep projection.  A lone 4096-wide projection runs level with hipBLASLt; the feed-forward
# pair goes through the kernel as one unit (fc1 with the GELU fused and a packed output
# that fc2 reads without re-ordering).
LINEAR_K_MULTIPLE = 256
LINEAR_MAX_IN = 4096
LINEAR_MAX_OUT = 3072
# Up to 512 rows (continuous batching's larger steps, Florence-2 beam batches), timed the
# same way: at 320 / 384 / 448 / 512 rows a 1024 x 1024 projection 6.3-6.9 against
# 10.8-11.1 us, fc2's shape 12.7-14.9 against 15.3-15.9 us; q|k|v 11.0 / 12.2 / 14.1 /
# 14.7 against 11.9 / 12.9 / 12.9 / 12.9 us and fc1 + GELU 14.7-20.1 against 12.7-13.2
# us plus the separate GELU.  With every projection of a layer on the kernel its
# LayerNorms stay deferred (three launches fewer per layer), which outweighs the q|k|v
# and fc1 shortfall at 448-512 rows.
LINEAR_MAX_ROWS = 512


@torch.library.custom_op("vflorence_amd::add_layer_norm", mutates_args=())
def add_layer_norm(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor,
                   bias: torch.Tensor, eps: float) -> torch.Tensor:
    """``LayerNorm(x + residual) * weight + bias`` over the last dimension."""
    dev = _require_gpu(x, residual, weight, bias)
    dim = x.shape[-1]
    if residual.shape != x.shape or weight.shape != (dim,) or bias.shape != (dim,):
        raise ValueError("add_layer_norm: x and residual must match; weight / bias are [dim]")
    if len({x.dtype, residual.dtype, weight.dtype, bias.dtype}) != 1:
        raise ValueError("add_layer_norm: all tensors must share one dtype")
    x2 = x.reshape(-1, dim)
    r2 = residual.reshape(-1, dim)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    out = torch.empty(x2.shape, dtype=x.dtype, device=dev)
    check(lib.vfl_add_layer_norm(x2.data_ptr(), x2.stride(0), r2.data_ptr(), r2.stride(0),
                                 weight.contiguous().data_ptr(), bias.contiguous().data_ptr(),
                                 out.data_ptr(), out.stride(0), x2.shape[0], dim, eps,
                                 _dtype_code(x.dtype), _stream(dev)))
    return out.view(x.shape)


@add_layer_norm.register_fake
def _(x, residual, weight, bias, eps):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op("vflorence_amd::embed_layer_norm", mutates_args=())
def embed_layer_norm(ids: torch.Tensor, positions: torch.Tensor, token_table: torch.Tensor,
                     token_scale: float, position_table: torch.Tensor, position_offset: int,
                     weight: torch.Tensor, bias: torch.Tensor, eps: float) -> torch.Tensor:
    """``LayerNorm(position_table[positions + position_offset] + token_table[ids] *
    token_scale) * weight + bias`` for int64 ``ids`` / ``positions`` [rows]: the decoder's
    embeddings and their LayerNorm in one launch, with ``add_layer_norm``'s arithmetic on
    the two looked-up rows (the scaled token row rounded to the element type first).  A
    row whose index lies outside its table comes out NaN."""
    dev = _require_gpu(ids, positions, token_table, position_table, weight, bias)
    dim = token_table.shape[-1]
    if (token_table.dim() != 2 or position_table.dim() != 2 or position_table.shape[1] != dim
            or weight.shape != (dim,) or bias.shape != (dim,)):
        raise ValueError("embed_layer_norm: tables must be [rows, dim]; weight / bias [dim]")
    if ids.dtype != torch.int64 or positions.dtype != torch.int64 or ids.dim() != 1 \
            or positions.shape != ids.shape:
        raise ValueError("embed_layer_norm: ids and positions must be int64 [rows]")
    if len({token_table.dtype, position_table.dtype, weight.dtype, bias.dtype}) != 1:
        raise ValueError("embed_layer_norm: tables, weight and bias must share one dtype")
    tok = token_table if token_table.stride(-1) == 1 else token_table.contiguous()
    pos = position_table if position_table.stride(-1) == 1 else position_table.contiguous()
    ids, positions = ids.contiguous(), positions.contiguous()
    rows = ids.shape[0]
    out = torch.empty(rows, dim, dtype=tok.dtype, device=dev)
    check(lib.vfl_embed_layer_norm(
        ids.data_ptr(), positions.data_ptr(), rows, tok.data_ptr(), tok.shape[0], tok.stride(0),
        token_scale, pos.data_ptr(), pos.shape[0], pos.stride(0), position_offset,
        weight.contiguous().data_ptr(), bias.contiguous().data_ptr(), out.data_ptr(),
        out.stride(0), dim, eps, _dtype_code(tok.dtype), _stream(dev)))
    return out


@embed_layer_norm.register_fake
def _(ids, positions, token_table, token_scale, position_table, position_offset, weight, bias,
      eps):
    return token_table.new_empty(ids.shape[0], token_table.shape[-1])


def linear_fits(rows: int, weight: torch.Tensor, *, max_in: int | None = LINEAR_MAX_IN,
                max_out: int | None = LINEAR_MAX_OUT) -> bool:
    """Whether ``linear`` serves ``rows`` rows times ``weight``: a contiguous, 16-byte
    aligned 16-bit device weight, in_features a multiple of 256, at most 512 rows, and
    in / out features within ``max_in`` / ``max_out`` (None: no bound; the defaults are
    where a lone projection beats hipBLASLt -- the feed-forward pair, which fuses its
    activation, lifts them)."""
    out_features, in_features = weight.shape
    return (weight.is_cuda and weight.dtype in (torch.bfloat16, torch.float16)
            and weight.is_contiguous() and weight.data_ptr() % 16 == 0
            and 0 < rows <= LINEAR_MAX_ROWS and in_features % LINEAR_K_MULTIPLE == 0
            and (max_in is None or in_features <= max_in)
            and (max_out is None or out_features <= max_out))


def pack_linear_weight(weight: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """``weight`` ([out, in], 16-bit, on the GPU) re-laid out in the matrix cores' operand
    order for ``linear`` (1 KB blocks of 16 rows x 32 inputs in lane order, rows padded
    to a multiple of 32): a 1-D tensor of the same dtype, new or ``out`` (rewritten in
    place, so HIP graphs captured over it read the new values)."""
    dev = _require_gpu(weight)
    out_features, in_features = weight.shape
    w = weight.contiguous()
    elems = max(1, lib.vfl_linear_packed_elems(out_features, in_features))
    if out is not None:
        if out.shape != (elems,) or out.dtype != weight.dtype or out.device != weight.device:
            raise ValueError(f"out must be a {weight.dtype} tensor of {elems} elements on "
                             f"{weight.device}")
        packed = out
    else:
        packed = torch.empty(elems, dtype=weight.dtype, device=dev)
    check(lib.vfl_pack_linear_weight(w.data_ptr(), w.stride(0), out_features, in_features,
                                     packed.data_ptr(), _dtype_code(weight.dtype), _stream(dev)))
    return packed


# vfl_linear flags (include/vflorence_amd.h)
LINEAR_GELU, LINEAR_X_PACKED, LINEAR_Y_PACKED = 1, 2, 4


def packed_elems(rows: int, cols: int) -> int:
    """Elements of a packed [rows, cols] array (rows padded to a multiple of 32)."""
    return (rows + 31) // 32 * 32 * cols


@torch.library.custom_op("vflorence_amd::linear", mutates_args=())
def linear(x: torch.Tensor, packed_weight: torch.Tensor, bias: torch.Tensor | None,
           out_features: int, rows: int = -1, flags: int = 0) -> torch.Tensor:
    """``act(x @ weight.T + bias)`` (nn.Linear, then GELU with ``LINEAR_GELU``), fp32
    sums, with the weight given as ``pack_linear_weight(weight)``.  ``x`` is ``[..., in]``,
    or with ``LINEAR_X_PACKED`` the packed output of an earlier call for ``rows`` rows.
    The result is ``[..., out_features]``, or with ``LINEAR_Y_PACKED`` a packed 1-D
    activation for the next call."""
    dev = _require_gpu(x, packed_weight) if bias is None else _require_gpu(x, packed_weight,
                                                                          bias)
    padded_out = (out_features + 31) // 32 * 32
    if out_features <= 0 or packed_weight.dim() != 1 or packed_weight.numel() % padded_out:
        raise ValueError(f"linear: packed_weight does not hold a packed [{out_features}, in] "
                         "weight")
    in_features = packed_weight.numel() // padded_out
    if bias is not None and bias.shape != (out_features,):
        raise ValueError("linear: bias must be [out_features]")
    if x.dtype != packed_weight.dtype or (bias is not None and bias.dtype != x.dtype):
        raise ValueError("linear: x, weight and bias must share one dtype")
    if flags & LINEAR_X_PACKED:
        if rows <= 0 or x.dim() != 1 or x.numel() != packed_elems(rows, in_features):
            raise ValueError(f"linear: x is not a packed [{rows}, {in_features}] activation")
        x2, lead = x, (rows,)
    else:
        if x.shape[-1] != in_features:
            raise ValueError(f"linear: x has {x.shape[-1]} features, the weight {in_features}")
        x2 = x.reshape(-1, in_features)
        if x2.stride(-1) != 1 or x2.stride(0) % 8 or x2.data_ptr() % 16:
            x2 = x2.contiguous()
        rows, lead = x2.shape[0], x.shape[:-1]
    b = None if bias is None else bias.contiguous()
    if flags & LINEAR_Y_PACKED:
        out = torch.empty(packed_elems(rows, out_features), dtype=x.dtype, device=dev)
        y_stride = 0
    else:
        out = torch.empty(rows, out_features, dtype=x.dtype, device=dev)
        y_stride = out.stride(0)
    x_stride = 0 if flags & LINEAR_X_PACKED else x2.stride(0)
    check(lib.vfl_linear(x2.data_ptr(), x_stride, packed_weight.data_ptr(),
                         None if b is None else b.data_ptr(), out.data_ptr(), y_stride, rows,
                         out_features, in_features, flags, _dtype_code(x.dtype), _stream(dev)))
    return out if flags & LINEAR_Y_PACKED else out.view(*lead, out_features)


@linear.register_fake
def _(x, packed_weight, bias, out_features, rows=-1, flags=0):
    if flags & LINEAR_Y_PACKED:
        n = rows if flags & LINEAR_X_PACKED else x.numel() // x.shape[-1]
        return x.new_empty(packed_elems(n, out_features))
    lead = (rows,) if flags & LINEAR_X_PACKED else x.shape[:-1]
    return x.new_empty(*lead, out_features)


# Deferred LayerNorm (vfl_linear_residual / vfl_linear_norm / vfl_layer_norm_apply): a
# post-LN sublayer's output h' = LN(v) travels as the pre-norm sum v and per-row,
# per-32-feature (mean, sum of squared deviations) statistics; its consumers fold the
# LayerNorm into their weights and finish it in their epilogue.
STAT_TILE = 32


def fold_layer_norm(weight: torch.Tensor, bias: torch.Tensor | None, gamma: torch.Tensor,
                    beta: torch.Tensor, out: tuple | None = None) -> tuple:
    """The operands of ``linear_norm`` for ``linear(LN(v))`` with this LayerNorm's
    ``gamma`` / ``beta``: the packed ``W' = rnd(W diag(gamma))``, ``u = sum_k W'[:, k]``
    and ``b' = bias + W beta`` (both fp32).  With ``out`` (an earlier result of the same
    shapes) they are rewritten in place, so HIP graphs captured over them stay valid."""
    _require_gpu(weight, gamma, beta)
    if gamma.shape != (weight.shape[1],) or beta.shape != gamma.shape:
        raise ValueError("fold_layer_norm: gamma / beta must be [in_features]")
    with torch.no_grad():
        w32 = weight.float()
        folded = (w32 * gamma.float()).to(weight.dtype)
        u = folded.float().sum(dim=1)
        fb = w32 @ beta.float()
        if bias is not None:
            fb = fb + bias.float()
        if out is None:
            return pack_linear_weight(folded), u, fb
        packed, u_out, fb_out = out
        pack_linear_weight(folded, out=packed)
        u_out.copy_(u)
        fb_out.copy_(fb)
        return out


def _stats_shape(rows: int, features: int) -> tuple:
    return (rows, features // STAT_TILE, 2)


@torch.library.custom_op("vflorence_amd::linear_residual", mutates_args=())
def linear_residual(x: torch.Tensor, packed_weight: torch.Tensor, bias: torch.Tensor | None,
                    residual: torch.Tensor, r_stats: torch.Tensor | None,
                    r_gamma: torch.Tensor | None, r_beta: torch.Tensor | None, r_eps: float,
                    out_features: int, rows: int = -1,
                    flags: int = 0) -> tuple[torch.Tensor, torch.Tensor]:
    """A post-LN sublayer's output projection: ``v = rnd(rnd(x @ W.T + bias) + h)`` with
    h = ``residual`` (r_stats None) or LN(residual) under r_stats / r_gamma / r_beta /
    r_eps, and v's tile statistics.  x is ``[rows, in]`` (or, with ``LINEAR_X_PACKED``, a
    packed activation of ``rows`` rows); residual and v are ``[rows, out_features]``."""
    dev = _require_gpu(x, packed_weight, residual,
                       *(t for t in (bias, r_stats, r_gamma, r_beta) if t is not None))
    padded_out = (out_features + 31) // 32 * 32
    if (out_features <= 0 or out_features % STAT_TILE or packed_weight.dim() != 1
            or packed_weight.numel() % padded_out):
        raise ValueError("linear_residual: packed_weight must hold a packed [out, in] weight "
                         f"with out a multiple of {STAT_TILE}")
    in_features = packed_weight.numel() // padded_out
    if flags & ~LINEAR_X_PACKED:
        raise ValueError("linear_residual: only LINEAR_X_PACKED applies")
    if flags & LINEAR_X_PACKED:
        if rows <= 0 or x.dim() != 1 or x.numel() != packed_elems(rows, in_features):
            raise ValueError(f"linear_residual: x is not a packed [{rows}, {in_features}] "
                             "activation")
        x2, x_stride = x, 0
    else:
        if x.dim() != 2 or x.shape[1] != in_features:
            raise ValueError(f"linear_residual: x must be [rows, {in_features}]")
        x2 = x if x.stride(-1) == 1 and x.stride(0) % 8 == 0 and x.data_ptr() % 16 == 0 \
            else x.contiguous()
        rows, x_stride = x2.shape[0], x2.stride(0)
    if residual.shape != (rows, out_features) or residual.stride(-1) != 1:
        raise ValueError(f"linear_residual: residual must be [{rows}, {out_features}], unit "
                         "stride")
    if residual.stride(0) % 4 or residual.data_ptr() % 8:
        residual = residual.contiguous()
    dt = x.dtype
    if packed_weight.dtype != dt or residual.dtype != dt or (bias is not None
                                                             and bias.dtype != dt):
        raise ValueError("linear_residual: x, weight, bias and residual must share one dtype")
    if bias is not None and bias.shape != (out_features,):
        raise ValueError("linear_residual: bias must be [out_features]")
    if r_stats is not None:
        if (r_gamma is None or r_beta is None or r_stats.dtype != torch.float32
                or r_stats.shape != _stats_shape(rows, out_features)
                or not r_stats.is_contiguous() or r_gamma.shape != (out_features,)
                or r_beta.shape != (out_features,) or r_gamma.dtype != dt
                or r_beta.dtype != dt):
            raise ValueError("linear_residual: r_stats [rows, out/32, 2] float32 and gamma / "
                             "beta [out] of x's dtype describe a deferred residual")
    v = torch.empty(rows, out_features, dtype=dt, device=dev)
    stats = torch.empty(_stats_shape(rows, out_features), dtype=torch.float32, device=dev)
    g = None if r_gamma is None else r_gamma.contiguous()
    b = None if r_beta is None else r_beta.contiguous()
    check(lib.vfl_linear_residual(
        x2.data_ptr(), x_stride, packed_weight.data_ptr(),
        None if bias is None else bias.contiguous().data_ptr(), residual.data_ptr(),
        residual.stride(0), None if r_stats is None else r_stats.data_ptr(),
        None if g is None else g.data_ptr(), None if b is None else b.data_ptr(), r_eps,
        v.data_ptr(), v.stride(0), stats.data_ptr(), rows, out_features, in_features, flags,
        _dtype_code(dt), _stream(dev)))
    return v, stats


@linear_residual.register_fake
def _(x, packed_weight, bias, residual, r_stats, r_gamma, r_beta, r_eps, out_features,
      rows=-1, flags=0):
    n = rows if flags & LINEAR_X_PACKED else x.shape[0]
    return (x.new_empty(n, out_features),
            x.new_empty(_stats_shape(n, out_features), dtype=torch.float32))


@torch.library.custom_op("vflorence_amd::linear_norm", mutates_args=())
def linear_norm(x: torch.Tensor, x_stats: torch.Tensor, eps: float,
                packed_weight: torch.Tensor, u: torch.Tensor, folded_bias: torch.Tensor,
                out_features: int, flags: int = 0) -> torch.Tensor:
    """``act(LN(x) @ W.T + bias)`` for a pre-norm sum x ``[rows, in]`` with its tile
    statistics, given ``fold_layer_norm``'s operands (LN's eps here); ``LINEAR_GELU``
    and ``LINEAR_Y_PACKED`` as for ``linear``."""
    dev = _require_gpu(x, x_stats, packed_weight, u, folded_bias)
    padded_out = (out_features + 31) // 32 * 32
    if out_features <= 0 or packed_weight.dim() != 1 or packed_weight.numel() % padded_out:
        raise ValueError(f"linear_norm: packed_weight does not hold a packed [{out_features}, "
                         "in] weight")
    in_features = packed_weight.numel() // padded_out
    if flags & ~(LINEAR_GELU | LINEAR_Y_PACKED):
        raise ValueError("linear_norm: only LINEAR_GELU and LINEAR_Y_PACKED apply")
    if x.dim() != 2 or x.shape[1] != in_features or x.stride(-1) != 1 or x.stride(0) % 8 \
            or x.data_ptr() % 16:
        raise ValueError(f"linear_norm: x must be [rows, {in_features}], unit stride, 16-byte "
                         "aligned rows")
    rows = x.shape[0]
    if (x_stats.dtype != torch.float32 or x_stats.shape != _stats_shape(rows, in_features)
            or not x_stats.is_contiguous()):
        raise ValueError("linear_norm: x_stats must be [rows, in/32, 2] float32")
    if (u.shape != (out_features,) or folded_bias.shape != (out_features,)
            or u.dtype != torch.float32 or folded_bias.dtype != torch.float32):
        raise ValueError("linear_norm: u / folded_bias must be [out_features] float32")
    if packed_weight.dtype != x.dtype:
        raise ValueError("linear_norm: x and the weight must share one dtype")
    if flags & LINEAR_Y_PACKED:
        out = torch.empty(packed_elems(rows, out_features), dtype=x.dtype, device=dev)
        y_stride = 0
    else:
        out = torch.empty(rows, out_features, dtype=x.dtype, device=dev)
        y_stride = out.stride(0)
    check(lib.vfl_linear_norm(x.data_ptr(), x.stride(0), x_stats.data_ptr(), eps,
                              packed_weight.data_ptr(), u.contiguous().data_ptr(),
                              folded_bias.contiguous().data_ptr(), out.data_ptr(), y_stride,
                              rows, out_features, in_features, flags, _dtype_code(x.dtype),
                              _stream(dev)))
    return out


@linear_norm.register_fake
def _(x, x_stats, eps, packed_weight, u, folded_bias, out_features, flags=0):
    if flags & LINEAR_Y_PACKED:
        return x.new_empty(packed_elems(x.shape[0], out_features))
    return x.new_empty(x.shape[0], out_features)


@torch.library.custom_op("vflorence_amd::layer_norm_apply", mutates_args=())
def layer_norm_apply(v: torch.Tensor, stats: torch.Tensor, gamma: torch.Tensor,
                     beta: torch.Tensor, eps: float) -> torch.Tensor:
    """LN(v) from v's tile statistics (v ``[rows, dim]``, dim a multiple of 32)."""
    dev = _require_gpu(v, stats, gamma, beta)
    rows, dim = v.shape
    if (stats.dtype != torch.float32 or stats.shape != _stats_shape(rows, dim)
            or not stats.is_contiguous() or gamma.shape != (dim,) or beta.shape != (dim,)
            or gamma.dtype != v.dtype or beta.dtype != v.dtype):
        raise ValueError("layer_norm_apply: stats [rows, dim/32, 2] float32, gamma / beta [dim] "
                         "of v's dtype")
    v2 = v if v.stride(-1) == 1 and v.stride(0) % 4 == 0 and v.data_ptr() % 8 == 0 \
        else v.contiguous()
    out = torch.empty(rows, dim, dtype=v.dtype, device=dev)
    check(lib.vfl_layer_norm_apply(v2.data_ptr(), v2.stride(0), stats.data_ptr(),
                                   gamma.contiguous().data_ptr(), beta.contiguous().data_ptr(),
                                   eps, out.data_ptr(), out.stride(0), rows, dim,
                                   _dtype_code(v.dtype), _stream(dev)))
    return out


@layer_norm_apply.register_fake
def _(v, stats, gamma, beta, eps):
    return v.new_empty(v.shape)


class TopkRules:
    """The history-free generation rules of one SamplingParams, packed for the kernel:
    a device int32 array ``[eos | suppressed | begin-suppressed | forced BOS | forced EOS]``
    and the length thresholds (see LogitsProcessor for their meaning)."""

    def __init__(self, *, eos, suppress, begin_suppress, forced_bos, forced_eos, min_length: int,
                 max_length: int, begin_index: int, device):
        lists = [list(t) for t in (eos, suppress, begin_suppress, forced_bos, forced_eos)]
        self.counts = [len(t) for t in lists]
        flat = [t for lst in lists for t in lst]
        self.tokens = (torch.tensor(flat, dtype=torch.int32, device=device) if flat else None)
        self.min_length = min_length if lists[0] else 0
        self.max_length, self.begin_index = max_length, begin_index


def logprob_topk(logits: torch.Tensor, k: int, *, log_softmax: bool,
                 lengths: torch.Tensor | None = None, rules: TopkRules | None = None,
                 out: tuple[torch.Tensor, torch.Tensor] | None = None):
    """Per row: (log-softmax), generation rules, and the k best scores with their token
    ids, best first (ties: lower token id).  Returns (float32 [rows, k], int64 [rows, k]):
    new device tensors, or ``out`` filled in -- which may be pinned host tensors, written
    by the kernel itself (valid on the host once the stream has been synchronized)."""
    dev = _require_gpu(logits)
    if logits.dim() != 2 or logits.stride(1) != 1:
        raise ValueError("logits must be [rows, vocab] with contiguous rows")
    rows, vocab = logits.shape
    if not 1 <= k <= min(MAX_K, vocab):
        raise ValueError(f"k must be in [1, min({MAX_K}, vocab)], got {k}")
    counts = rules.counts if rules is not None else [0] * 5
    tokens = rules.tokens if rules is not None else None
    if sum(counts) and lengths is None:
        raise ValueError("the rules need per-row lengths")
    if lengths is not None and (lengths.dtype != torch.int64 or lengths.shape != (rows,)):
        raise ValueError("lengths must be int64 [rows]")
    if out is None:
        scores = torch.empty(rows, k, dtype=torch.float32, device=dev)
        ids = torch.empty(rows, k, dtype=torch.int64, device=dev)
    else:
        scores, ids = out
        for t, dt in ((scores, torch.float32), (ids, torch.int64)):
            if t.dtype != dt or t.shape != (rows, k) or not t.is_contiguous():
                raise ValueError(f"out tensors must be contiguous {dt} [{rows}, {k}]")
            if not (t.device == logits.device or (t.device.type == "cpu" and t.is_pinned())):
                raise ValueError("out tensors must be on the logits' device or in pinned "
                                 "host memory")
    check(lib.vfl_logprob_topk(
        logits.data_ptr(), logits.stride(0), rows, vocab, _dtype_code(logits.dtype),
        None if lengths is None else lengths.data_ptr(),
        None if tokens is None else tokens.data_ptr(),
        rules.min_length if rules else 0, rules.max_length if rules else 0,
        rules.begin_index if rules else -1, *counts, int(log_softmax), k, scores.data_ptr(),
        ids.data_ptr(), _stream(dev)))
    return scores, ids

