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
LINEAR_MAX_ROWS = 256


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


def linear_fits(rows: int, weight: torch.Tensor, *, max_in: int | None = LINEAR_MAX_IN,
                max_out: int | None = LINEAR_MAX_OUT) -> bool:
    """Whether ``linear`` serves ``rows`` rows times ``weight``: a contiguous, 16-byte
    aligned 16-bit device weight, in_features a multiple of 256, at most 256 rows, and
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
                 lengths: torch.Tensor | None = None, rules: TopkRules | None = None):
    """Per row: (log-softmax), generation rules, and the k best scores with their token
    ids, best first (ties: lower token id).  Returns (float32 [rows, k], int64 [rows, k])."""
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
    scores = torch.empty(rows, k, dtype=torch.float32, device=dev)
    ids = torch.empty(rows, k, dtype=torch.int64, device=dev)
    check(lib.vfl_logprob_topk(
        logits.data_ptr(), logits.stride(0), rows, vocab, _dtype_code(logits.dtype),
        None if lengths is None else lengths.data_ptr(),
        None if tokens is None else tokens.data_ptr(),
        rules.min_length if rules else 0, rules.max_length if rules else 0,
        rules.begin_index if rules else -1, *counts, int(log_softmax), k, scores.data_ptr(),
        ids.data_ptr(), _stream(dev)))
    return scores, ids

