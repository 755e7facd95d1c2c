"""Torch-facing wrappers of the gfx950 C ABI: the counterpart of ``vllm_cpu_attn``.

The reference reaches its attention arithmetic through four functions of the external
``vllm_cpu_attn`` package (vflorence/layers/attention.py:18,55,61,98;
vflorence/engine/model_runner.py:38,252,308).  This module offers the same four names
with the same keyword arguments, plus ``copy_blocks`` for the copy-on-write loop of
vflorence/engine/model_runner.py:162-167.  Every call validates shapes on the host,
then enqueues HIP kernels on torch's current stream of the tensors' device.  CPU
tensors are rejected: there is no host implementation behind these names.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import torch

from . import _lib
from ._lib import SchedMeta, check, lib

_DTYPE_CODES = {
    torch.float32: _lib.VFL_FLOAT32,
    torch.bfloat16: _lib.VFL_BFLOAT16,
    torch.float16: _lib.VFL_FLOAT16,
}

# Head sizes with a compiled kernel: the reference's list (vflorence/layers/attention.py:6).
SUPPORTED_HEAD_DIMS = frozenset({32, 48, 64, 80, 96, 112, 128, 160, 192, 224, 256, 512})
# Head sizes with every kernel built: beam groups keeping their own tables, the group
# plan and the fused KV write (BART and Florence-2 use 64).  Other head sizes run one
# row (or one shared-table group) per workgroup with the KV write as its own launch;
# the entry points take the same arguments and fall back by themselves.
NATIVE_HEAD_DIMS = frozenset({64, 128})
# Pool block sizes: 16 (this build's engine), and 32, the reference's on x86
# (vflorence/config.py:42), read by the one-row kernels as two 16-token parts (beam
# groups, group plans and the fused KV write then fall back as for other head sizes).
SUPPORTED_BLOCK_SIZES = frozenset({16, 32})
MAX_GROUP_SIZE = 8
# Waves per workgroup for the fused KV-write + self-attention launch over contexts longer
# than FUSED_ONE_WAVE_BLOCKS blocks (measured, 256 ragged rows up to 1024 tokens, three
# pools in rotation: one / two / four / eight waves 102.0 / 96.1 / 95.3 / 119.0 us).
FUSED_WAVES = 4
FUSED_ONE_WAVE_BLOCKS = 4
# Waves per workgroup of the fused launch over own-table row groups (beams): measured
# best from 1 to 8 blocks of context (64 x 4 beams, MI355X); more waves cost occupancy.
FUSED_GROUP_WAVES = 2


def v_tile_interleaved(dtype: torch.dtype) -> bool:
    """Whether V pools of ``dtype`` store each [block][head] slice token-interleaved.

    16-bit pools keep each block-head slice of V as [block_size/4][head_dim][4]: four
    consecutive tokens of one dim are adjacent, which is the reduction operand of the
    matrix-core kernel, and a token's head_dim values are 8 bytes apart.  fp32 pools
    keep the logical [block_size][head_dim] order.  The tensor shape is the reference's
    [num_blocks, H, block_size, head_dim] either way, and only this library's ops
    address the inside of a block (the reference leaves that layout to the attention
    backend: AGENTS.md section 5.3, "internal layout determined by the selected ISA").
    """
    return dtype != torch.float32


def v_cache_logical(v_cache: torch.Tensor) -> torch.Tensor:
    """V pool values in logical [NB, H, bs, D] (token, dim) order (a copy for 16-bit pools)."""
    if not v_tile_interleaved(v_cache.dtype):
        return v_cache
    nb, h, bs, d = v_cache.shape
    return v_cache.view(nb, h, bs // 4, d, 4).permute(0, 1, 2, 4, 3).reshape(nb, h, bs, d)


def v_cache_from_logical(v_logical: torch.Tensor) -> torch.Tensor:
    """A contiguous V pool (device layout) holding the given logical [NB, H, bs, D] values."""
    if not v_tile_interleaved(v_logical.dtype):
        return v_logical.contiguous()
    nb, h, bs, d = v_logical.shape
    return (v_logical.reshape(nb, h, bs // 4, 4, d).permute(0, 1, 2, 4, 3).contiguous()
            .view(nb, h, bs, d))


def _dtype_code(dtype: torch.dtype) -> int:
    try:
        return _DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; use float32, bfloat16 or float16") from None


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = tensors[0].device
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "vflorence_amd kernels need HIP device tensors; got a tensor on "
                f"{t.device} (there is no CPU path)"
            )
        if t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def get_isa(dtype: torch.dtype, block_size: int, head_dim: int) -> str:
    """The GPU target whose kernel serves (dtype, block_size, head_dim).

    Counterpart of ``vllm_cpu_attn.get_isa`` (vflorence/engine/model_runner.py:38);
    raises ValueError where the reference would have no ISA either.
    """
    isa = lib.vfl_get_isa(_dtype_code(dtype), int(block_size), int(head_dim))
    if isa is None:
        raise ValueError(
            f"no gfx950 kernel for dtype={dtype} block_size={block_size} head_dim={head_dim}; "
            f"supported head_dim {sorted(SUPPORTED_HEAD_DIMS)}, block_size "
            f"{sorted(SUPPORTED_BLOCK_SIZES)}"
        )
    return isa.decode()


def reshape_and_cache(
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    slot_mapping: torch.Tensor,
    isa: str | None = None,
) -> None:
    """``cache[slot // bs, h, slot % bs, :] = key[t, h, :]`` for K and V.

    Counterpart of ``vllm_cpu_attn.reshape_and_cache`` (vflorence/layers/attention.py:55-57,
    vflorence/engine/model_runner.py:252-259).  key/value are [T, H, D] with any token and
    head strides and a contiguous last dim; caches are contiguous [NB, H, bs, D]; slots
    are int64 [T].  Negative slots are skipped.  ``isa`` is accepted and ignored.
    """
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H, block_size, D] of one shape")
    num_blocks, num_heads, block_size, head_dim = k_cache.shape
    if block_size not in SUPPORTED_BLOCK_SIZES:
        raise ValueError(f"block_size={block_size} has no attention kernel; supported: "
                         f"{sorted(SUPPORTED_BLOCK_SIZES)}")
    dev = _require_gpu(key, value, k_cache, v_cache, slot_mapping)
    if key.dim() != 3 or value.shape != key.shape:
        raise ValueError(f"key/value must be [T, H, D] of one shape, got {key.shape}, {value.shape}")
    if key.shape[1:] != (num_heads, head_dim):
        raise ValueError(f"key is {tuple(key.shape)} but caches hold H={num_heads}, D={head_dim}")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if key.stride(-1) != 1 or value.stride(-1) != 1:
        raise ValueError("key/value need a contiguous last dimension")
    if not (key.dtype == value.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("key, value and caches must share one dtype")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (key.shape[0],):
        raise ValueError(f"slot_mapping must be int64 [{key.shape[0]}], got "
                         f"{slot_mapping.dtype} {tuple(slot_mapping.shape)}")
    if not slot_mapping.is_contiguous():
        slot_mapping = slot_mapping.contiguous()
    check(
        lib.vfl_reshape_and_cache(
            key.data_ptr(), value.data_ptr(), key.stride(0), key.stride(1), value.stride(0),
            value.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(),
            key.shape[0], num_heads, head_dim, block_size, num_blocks, _dtype_code(key.dtype),
            _stream(dev),
        )
    )


@dataclass(eq=False)
class GroupPlan:
    """A decode step's schedule of own-table row groups (``build_group_plan``): per
    dispatch slot, a group's first row and row count and, position by position, the
    distinct block ids its rows read with the rows that read each.  Made on the host
    from the step's block tables once; every layer's self-attention launch reads it
    (from the device copy) instead of walking the tables.

    ``words``: int32 [4 + slots * stride]; ``max_blocks``: the block-table width it was
    made for.
    """

    words: torch.Tensor
    stride: int
    slots: int
    max_blocks: int
    # copy-on-write pairs folded in (fold_plan_copies): for the fused launch only
    folded: bool = False

    def to(self, device, non_blocking: bool = False) -> "GroupPlan":
        return GroupPlan(self.words.to(device, non_blocking=non_blocking), self.stride,
                         self.slots, self.max_blocks, self.folded)


def group_plan_stride(max_group_size: int, max_blocks: int) -> int:
    """int32 words of one slot of a group plan (``vfl_group_plan_stride``)."""
    stride = int(lib.vfl_group_plan_stride(int(max_group_size), int(max_blocks)))
    if stride <= 0:
        raise ValueError(f"no group plan for groups of {max_group_size} rows over tables "
                         f"{max_blocks} wide (at most {MAX_GROUP_SIZE} rows, 65536 blocks)")
    return stride


def build_group_plan(block_table: torch.Tensor, seq_lens: torch.Tensor,
                     group_start: torch.Tensor, *, group_order: torch.Tensor | None = None,
                     num_slots: int | None = None, max_group_size: int = MAX_GROUP_SIZE,
                     block_size: int = 16, num_blocks: int | None = None,
                     out: torch.Tensor | None = None) -> GroupPlan:
    """Group plan of one step from host (CPU int32) tensors: the block table
    [rows, width], seq_lens [rows], group_start [groups + 1] and the optional dispatch
    order [groups] of the self-attention call it is for (``vfl_build_group_plan``).
    ``num_slots`` (default: the group count) sizes it for a launch padded to more
    groups; ``out`` reuses a CPU int32 buffer (pinned, say) of at least the size."""
    for name, t in (("block_table", block_table), ("seq_lens", seq_lens),
                    ("group_start", group_start)):
        if t.device.type != "cpu" or t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous CPU int32 tensor")
    if block_table.dim() != 2 or seq_lens.shape != (block_table.shape[0],):
        raise ValueError("block_table must be [rows, width] and seq_lens [rows]")
    num_groups = group_start.numel() - 1
    if group_order is not None and (group_order.device.type != "cpu" or
                                    group_order.dtype != torch.int32 or
                                    group_order.shape != (num_groups,)):
        raise ValueError(f"group_order must be a CPU int32 tensor [{num_groups}]")
    slots = num_groups if num_slots is None else int(num_slots)
    width = block_table.shape[1]
    stride = group_plan_stride(max_group_size, width)
    words = 4 + slots * stride
    if out is None:
        out = torch.empty(words, dtype=torch.int32)
    elif out.device.type != "cpu" or out.dtype != torch.int32 or out.numel() < words:
        raise ValueError(f"out must be a CPU int32 tensor of at least {words} words")
    check(lib.vfl_build_group_plan(
        block_table.data_ptr(), block_table.stride(0), width, seq_lens.data_ptr(),
        block_table.shape[0], group_start.data_ptr(),
        None if group_order is None else group_order.data_ptr(), num_groups, block_size,
        (1 << 62) if num_blocks is None else int(num_blocks), out.data_ptr(), slots, stride))
    return GroupPlan(out[:words], stride, slots, width)


def slot_descriptor_stride(max_blocks: int) -> int:
    """int32 words of one slot descriptor over block tables ``max_blocks`` wide."""
    stride = int(lib.vfl_slot_descriptor_stride(int(max_blocks)))
    if stride <= 0:
        raise ValueError(f"no slot descriptors for tables {max_blocks} wide")
    return stride


def build_slot_descriptors(block_table: torch.Tensor, seq_lens: torch.Tensor,
                           group_start: torch.Tensor, *, group_order: torch.Tensor | None = None,
                           num_slots: int | None = None,
                           out: torch.Tensor | None = None) -> GroupPlan:
    """Slot descriptors of shared-table groups (``vfl_build_slot_descriptors``) from host
    CPU int32 tensors: per dispatch slot, the group's first row, rows, length and table
    row, so a cross-attention workgroup reads its group in one load level.  Pass the
    device copy as ``get_scheduler_metadata(slot_descriptors=...)``.  ``num_slots``
    (default: the group count) sizes it for a launch padded to more groups; ``out``
    reuses a CPU int32 buffer of at least the size."""
    for name, t in (("block_table", block_table), ("seq_lens", seq_lens),
                    ("group_start", group_start)):
        if t.device.type != "cpu" or t.dtype != torch.int32 or not t.is_contiguous():
            raise ValueError(f"{name} must be a contiguous CPU int32 tensor")
    if block_table.dim() != 2 or seq_lens.shape != (block_table.shape[0],):
        raise ValueError("block_table must be [rows, width] and seq_lens [rows]")
    num_groups = group_start.numel() - 1
    if group_order is not None and (group_order.device.type != "cpu" or
                                    group_order.dtype != torch.int32 or
                                    group_order.shape != (num_groups,)):
        raise ValueError(f"group_order must be a CPU int32 tensor [{num_groups}]")
    slots = num_groups if num_slots is None else int(num_slots)
    width = block_table.shape[1]
    stride = slot_descriptor_stride(width)
    words = slots * stride
    if out is None:
        out = torch.empty(max(words, 4), dtype=torch.int32)
    elif out.device.type != "cpu" or out.dtype != torch.int32 or out.numel() < words:
        raise ValueError(f"out must be a CPU int32 tensor of at least {words} words")
    check(lib.vfl_build_slot_descriptors(
        block_table.data_ptr(), block_table.stride(0), width, seq_lens.data_ptr(),
        block_table.shape[0], group_start.data_ptr(),
        None if group_order is None else group_order.data_ptr(), num_groups, out.data_ptr(),
        slots, stride))
    return GroupPlan(out[:max(words, 4)], stride, slots, width)


def fold_plan_copies(plan: GroupPlan, src, dst, *, num_blocks: int) -> bool:
    """Fold a step's copy-on-write pairs ``src[i] -> dst[i]`` (host int64 sequences)
    into a host group plan (``vfl_fold_plan_copies``): the fused self-attention launch
    reading it then copies each pair's block for its layer's pools and the step needs no
    ``copy_blocks``.  Returns False, leaving the plan unchanged, when the pairs cannot
    be folded (a destination that is not one row's private block of the plan, say);
    the caller then copies them itself.  A folded plan names the sources in place of
    the fork blocks, so only ``self_attention_with_kv_write`` may read it."""
    import numpy as np

    if plan.words.device.type != "cpu":
        raise ValueError("fold_plan_copies works on the host copy of a plan")
    s = np.ascontiguousarray(src, dtype=np.int64)
    d = np.ascontiguousarray(dst, dtype=np.int64)
    if s.shape != d.shape or s.ndim != 1:
        raise ValueError("src and dst must be 1-D sequences of one length")
    rc = lib.vfl_fold_plan_copies(plan.words.data_ptr(), plan.slots, plan.stride,
                                  s.ctypes.data, d.ctypes.data, s.size, int(num_blocks))
    if rc == _lib.VFL_OK and s.size:
        plan.folded = True
    return rc == _lib.VFL_OK


def plan_copies_supported(dtype: torch.dtype, head_dim: int, block_size: int) -> bool:
    """Whether the fused self-attention launch acts on a plan's copy sources for pools of
    this dtype, head size and block size (the matrix-core group kernel: 16-bit caches,
    head size 64 or 128, 16-token blocks); elsewhere the pairs are copied by
    ``copy_blocks``."""
    return dtype in (torch.bfloat16, torch.float16) and head_dim in (64, 128) and block_size == 16


@dataclass(eq=False)
class SchedulerMetadata:
    """Launch plan for ``attention_with_kv_cache``: the GPU stand-in for the opaque
    tensor ``vllm_cpu_attn.get_scheduler_metadata`` returns.

    ``group_start`` (device int32 [num_groups + 1]) lists row groups -- the beams of a
    request.  Without ``own_tables`` a group's rows share one block-table row and
    length (cross-attention over one encoder page list) and its K/V is read once.  With
    ``own_tables`` every row keeps its own table and length, and a block that several
    rows of a group list at the same position is read once for all of them (decoder
    self-attention, where copy-on-write forks share prefix blocks); any partition of
    the rows gives the same results.  ``group_order`` (device int32 [num_groups]) is
    the dispatch order, longest context first.  The launch shape is fixed at call time
    from the block table's width, which the host always knows, so no device value is
    read back.
    """

    num_heads: int
    head_dim: int
    block_size: int
    dtype: torch.dtype
    group_start: torch.Tensor | None = None
    group_order: torch.Tensor | None = None
    num_groups: int | None = None
    max_group_size: int = 1
    waves_per_workgroup: int = 0
    own_tables: bool = False
    # Groups that do work when the launch holds more group slots (fixed-address staging:
    # unused slots exit at once); the default wave count is chosen for these.
    active_groups: int | None = None
    # The caller's promise that each row writes its new token at the slot of its last
    # context position, in a block no other row reads (the block manager's
    # copy-on-write invariant); lets the self-attention op fuse the KV write.
    fuse_kv_write: bool = False
    # Device copy of the step's group plan (own-table groups, 16-bit caches): the
    # launch reads the groups' blocks from it instead of walking the tables.
    group_plan: GroupPlan | None = None
    # Device copy of slot descriptors (shared-table groups, build_slot_descriptors): the
    # launch reads each slot's group, length and table row from it in one load level.
    slot_descriptors: GroupPlan | None = None
    _plans: dict = field(default_factory=dict, repr=False)

    def plan(self, num_rows: int, max_blocks: int) -> SchedMeta:
        key = (num_rows, max_blocks)
        meta = self._plans.get(key)
        if meta is None:
            meta = SchedMeta()
            groups = num_rows if self.group_start is None else self.num_groups
            waves = self.waves_per_workgroup
            if waves == 0 and self.fuse_kv_write:
                if self.own_tables and self.group_start is not None:
                    waves = FUSED_GROUP_WAVES
                else:
                    # measured best for the fused write + attention kernel (MI355X, bf16,
                    # 256 rows x 16 heads): one wave up to 4 blocks of context (a decode
                    # step's short contexts are latency-bound; more waves only add a
                    # merge), two beyond (ragged contexts up to 1024 tokens)
                    waves = 1 if max_blocks <= FUSED_ONE_WAVE_BLOCKS else FUSED_WAVES
            elif waves == 0 and self.active_groups is not None:
                # the library's default for a launch of just the working groups
                active = max(1, min(self.active_groups, groups))
                probe = SchedMeta()
                check(
                    lib.vfl_get_scheduler_metadata(
                        active, active, self.num_heads, self.head_dim, self.block_size,
                        max_blocks, self.max_group_size, _dtype_code(self.dtype), 0,
                        _lib.VFL_GROUP_OWN_TABLES if self.own_tables
                        else _lib.VFL_GROUP_SHARED_TABLE,
                        ctypes.byref(probe),
                    )
                )
                waves = probe.waves_per_workgroup
            check(
                lib.vfl_get_scheduler_metadata(
                    num_rows, groups, self.num_heads, self.head_dim, self.block_size,
                    max_blocks, self.max_group_size, _dtype_code(self.dtype), waves,
                    _lib.VFL_GROUP_OWN_TABLES if self.own_tables else _lib.VFL_GROUP_SHARED_TABLE,
                    ctypes.byref(meta),
                )
            )
            gp = self.group_plan if self.group_plan is not None else self.slot_descriptors
            if gp is not None:
                if gp.max_blocks != max_blocks:
                    raise ValueError(f"the group plan was made for block tables {gp.max_blocks} "
                                     f"wide, the call's table is {max_blocks} wide")
                meta.group_plan = gp.words.data_ptr()
                meta.group_plan_stride = gp.stride
                meta.group_plan_slots = gp.slots
            self._plans[key] = meta
        return meta


def longest_first(lengths) -> list[int]:
    """Group indices sorted by descending length (stable): the dispatch order that
    starts the longest contexts first so the short ones fill the tail."""
    return sorted(range(len(lengths)), key=lambda i: -int(lengths[i]))


def balanced_order(lengths, run: int) -> list[int]:
    """``longest_first`` with every other run of ``run`` groups reversed.

    For a launch whose workgroups are all resident at once (cross-attention: one per
    group and head).  Workgroups go to the 8 XCDs in turn and, inside an XCD, to its CUs
    in turn.  So with H heads a CU receives the groups at order positions p, p + run,
    p + 2 run, ... where run = CUs // H.  Sorted longest first, the CU taking p = 0
    would then hold the longest group of every run.  Reversing alternate runs pairs
    long with short on each CU.  Measured with 64 groups x 16 heads on MI355X's 256 CUs
    (run 16): 32.75 us against 33.2 us.
    """
    order = longest_first(lengths)
    run = max(1, int(run))
    out = []
    for i in range(0, len(order), run):
        chunk = order[i:i + run]
        out += chunk[::-1] if (i // run) % 2 else chunk
    return out


_cu_count: dict[int, int] = {}


def resident_run(device, num_heads: int) -> int:
    """The ``balanced_order`` run for a launch of one workgroup per (group, head) on
    ``device``: its compute units divided by the heads."""
    idx = torch.device(device).index or 0
    if idx not in _cu_count:
        _cu_count[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return max(1, _cu_count[idx] // max(1, num_heads))


def get_scheduler_metadata(
    *,
    num_reqs: int,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    seq_lens: torch.Tensor | None = None,
    dtype: torch.dtype,
    query_start_loc: torch.Tensor | None = None,
    causal: bool = False,
    isa: str | None = None,
    block_size: int,
    group_start: torch.Tensor | None = None,
    group_order: torch.Tensor | None = None,
    max_group_size: int = 1,
    waves_per_workgroup: int = 0,
    fuse_kv_write: bool = False,
    own_tables: bool = False,
    group_plan: GroupPlan | None = None,
    active_groups: int | None = None,
    slot_descriptors: GroupPlan | None = None,
) -> SchedulerMetadata:
    """Counterpart of ``vllm_cpu_attn.get_scheduler_metadata`` (keyword names from
    vflorence/layers/attention.py:18-29 and vflorence/engine/model_runner.py:308-319).

    ``group_start``/``group_order``/``max_group_size``/``waves_per_workgroup``/
    ``own_tables``/``group_plan``/``active_groups`` are this library's additions.  ``seq_lens``, ``query_start_loc``, ``causal`` and ``isa`` are
    accepted for signature compatibility; the plan does not need them (callers that
    know the lengths on the host pass ``group_order`` instead).
    """
    if num_kv_heads != num_heads:
        raise ValueError("grouped-query attention is not supported (num_kv_heads != num_heads)")
    if head_dim not in SUPPORTED_HEAD_DIMS:
        raise ValueError(f"head_dim {head_dim} has no gfx950 kernel ({sorted(SUPPORTED_HEAD_DIMS)})")
    if block_size not in SUPPORTED_BLOCK_SIZES:
        raise ValueError(f"block_size {block_size} has no gfx950 kernel")
    if not 1 <= max_group_size <= MAX_GROUP_SIZE:
        raise ValueError(f"max_group_size must be in [1, {MAX_GROUP_SIZE}]")
    if waves_per_workgroup not in (0, 1, 2, 4, 8):
        raise ValueError("waves_per_workgroup must be 0 (default), 1, 2, 4 or 8")
    num_groups = num_reqs
    if group_start is not None:
        if group_start.dtype != torch.int32 or group_start.dim() != 1:
            raise ValueError("group_start must be a 1-D int32 tensor")
        num_groups = group_start.numel() - 1
    if group_order is not None:
        if group_order.dtype != torch.int32 or group_order.shape != (num_groups,):
            raise ValueError(f"group_order must be int32 [{num_groups}]")
    if group_plan is not None:
        if not own_tables or group_start is None:
            raise ValueError("a group plan needs own_tables row groups (group_start)")
        w = group_plan.words
        if (w.device.type != "cuda" or w.dtype != torch.int32 or not w.is_contiguous()
                or w.numel() < 4 + group_plan.slots * group_plan.stride
                or group_plan.slots < num_groups):
            raise ValueError("group_plan must be a device copy of build_group_plan's output "
                             f"with at least {num_groups} slots")
    if slot_descriptors is not None:
        if own_tables or group_start is None:
            raise ValueError("slot descriptors describe shared-table row groups (group_start, "
                             "own_tables=False)")
        w = slot_descriptors.words
        if (w.device.type != "cuda" or w.dtype != torch.int32 or not w.is_contiguous()
                or w.numel() < slot_descriptors.slots * slot_descriptors.stride
                or slot_descriptors.slots < num_groups):
            raise ValueError("slot_descriptors must be a device copy of build_slot_descriptors' "
                             f"output with at least {num_groups} slots")
    return SchedulerMetadata(
        num_heads=num_heads,
        head_dim=head_dim,
        block_size=block_size,
        dtype=dtype,
        group_start=group_start,
        group_order=group_order,
        num_groups=num_groups,
        max_group_size=max_group_size,
        waves_per_workgroup=waves_per_workgroup,
        fuse_kv_write=fuse_kv_write,
        own_tables=own_tables,
        group_plan=group_plan,
        active_groups=active_groups,
        slot_descriptors=slot_descriptors,
    )


def attention_with_kv_cache(
    query: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    out: torch.Tensor,
    query_start_loc: torch.Tensor | None,
    seq_lens: torch.Tensor,
    *,
    scale: float,
    causal: bool = False,
    block_table: torch.Tensor,
    scheduler_metadata: SchedulerMetadata | None = None,
) -> None:
    """One-query-per-sequence paged attention, written into ``out`` in place.

    Counterpart of ``vllm_cpu_attn.attention_with_kv_cache`` as the reference calls it
    (vflorence/layers/attention.py:61-72 and :98-109): row r attends to the first
    ``seq_lens[r]`` tokens of the pages ``block_table[r]`` lists.  ``query_start_loc``
    must describe one query per sequence (the reference always passes
    ``arange(N + 1)``, vflorence/engine/model_runner.py:306); with one query at the end of
    its context ``causal`` changes nothing.
    """
    dev = _require_gpu(query, k_cache, v_cache, out, seq_lens, block_table)
    if query.dim() != 3 or query.stride(-1) != 1:
        raise ValueError("query must be [N, H, D] with a contiguous last dimension")
    num_rows, num_heads, head_dim = query.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H, block_size, D] of one shape")
    num_blocks, cache_heads, block_size, cache_dim = k_cache.shape
    if (cache_heads, cache_dim) != (num_heads, head_dim):
        raise ValueError(
            f"query has H={num_heads}, D={head_dim} but the cache holds H={cache_heads}, "
            f"D={cache_dim}"
        )
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if not (query.dtype == k_cache.dtype == v_cache.dtype == out.dtype):
        raise ValueError("query, caches and out must share one dtype")
    if out.shape != query.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of query's shape")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (num_rows,):
        raise ValueError(f"seq_lens must be int32 [{num_rows}], got {seq_lens.dtype} "
                         f"{tuple(seq_lens.shape)}")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != num_rows:
        raise ValueError(f"block_table must be int32 [{num_rows}, max_blocks], got "
                         f"{block_table.dtype} {tuple(block_table.shape)}")
    if query_start_loc is not None and query_start_loc.numel() != num_rows + 1:
        raise ValueError("query_start_loc must hold num_seqs + 1 offsets (one query per sequence)")
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    if not seq_lens.is_contiguous():
        seq_lens = seq_lens.contiguous()
    sm = scheduler_metadata
    if sm is None:
        sm = get_scheduler_metadata(
            num_reqs=num_rows, num_heads=num_heads, num_kv_heads=num_heads, head_dim=head_dim,
            dtype=query.dtype, block_size=block_size,
        )
    if sm.group_start is not None:
        _require_gpu(query, sm.group_start)
    if sm.group_order is not None:
        _require_gpu(query, sm.group_order)
    if sm.group_plan is not None and sm.group_plan.folded:
        raise ValueError("a group plan with copy-on-write folded in names the copy sources in "
                         "place of the fork blocks: only self_attention_with_kv_write reads it")
    num_groups = num_rows if sm.group_start is None else sm.num_groups
    meta = sm.plan(num_rows, block_table.shape[1])
    check(
        lib.vfl_attention_with_kv_cache(
            query.data_ptr(), query.stride(0), query.stride(1), k_cache.data_ptr(),
            v_cache.data_ptr(), out.data_ptr(), seq_lens.data_ptr(), block_table.data_ptr(),
            block_table.stride(0),
            None if sm.group_start is None else sm.group_start.data_ptr(),
            None if sm.group_order is None else sm.group_order.data_ptr(),
            num_rows, num_groups, num_heads, head_dim, block_size, num_blocks, float(scale),
            _dtype_code(query.dtype), ctypes.byref(meta), _stream(dev),
        )
    )


def self_attention_with_kv_write(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    out: torch.Tensor,
    seq_lens: torch.Tensor,
    slot_mapping: torch.Tensor,
    *,
    scale: float,
    block_table: torch.Tensor,
    scheduler_metadata: SchedulerMetadata,
) -> None:
    """``reshape_and_cache`` + ``attention_with_kv_cache`` in one launch (the body of the
    reference's vflorence::self_attention op, vflorence/layers/attention.py:53-73).

    Only valid under ``scheduler_metadata.fuse_kv_write`` (see SchedulerMetadata); the
    op falls back to the two calls otherwise.
    """
    sm = scheduler_metadata
    if not sm.fuse_kv_write:
        raise ValueError("self_attention_with_kv_write needs metadata made with fuse_kv_write=True")
    if sm.group_start is not None and not sm.own_tables:
        raise ValueError("the fused self-attention path groups rows only with own_tables=True")
    dev = _require_gpu(query, key, value, k_cache, v_cache, out, seq_lens, slot_mapping,
                       block_table)
    if key.dim() != 3 or value.shape != key.shape or key.shape != query.shape:
        raise ValueError("query, key and value must be [N, H, D] of one shape")
    if key.stride(-1) != 1 or value.stride(-1) != 1 or query.stride(-1) != 1:
        raise ValueError("query/key/value need a contiguous last dimension")
    num_rows, num_heads, head_dim = query.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("k_cache/v_cache must be [num_blocks, H, block_size, D] of one shape")
    num_blocks, cache_heads, block_size, cache_dim = k_cache.shape
    if (cache_heads, cache_dim) != (num_heads, head_dim):
        raise ValueError("query/key shape does not match the caches")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise ValueError("caches must be contiguous")
    if not (query.dtype == key.dtype == value.dtype == k_cache.dtype == v_cache.dtype == out.dtype):
        raise ValueError("query, key, value, caches and out must share one dtype")
    if out.shape != query.shape or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of query's shape")
    if seq_lens.dtype != torch.int32 or seq_lens.shape != (num_rows,):
        raise ValueError(f"seq_lens must be int32 [{num_rows}]")
    if slot_mapping.dtype != torch.int64 or slot_mapping.shape != (num_rows,):
        raise ValueError(f"slot_mapping must be int64 [{num_rows}]")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != num_rows:
        raise ValueError(f"block_table must be int32 [{num_rows}, max_blocks]")
    if block_table.stride(1) != 1:
        block_table = block_table.contiguous()
    seq_lens = seq_lens.contiguous()
    slot_mapping = slot_mapping.contiguous()
    if sm.group_start is not None:
        _require_gpu(query, sm.group_start)
    if sm.group_order is not None:
        _require_gpu(query, sm.group_order)
    num_groups = num_rows if sm.group_start is None else sm.num_groups
    meta = sm.plan(num_rows, block_table.shape[1])
    check(
        lib.vfl_self_attention_with_kv_write(
            query.data_ptr(), query.stride(0), query.stride(1), key.data_ptr(), key.stride(0),
            key.stride(1), value.data_ptr(), value.stride(0), value.stride(1),
            slot_mapping.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), out.data_ptr(),
            seq_lens.data_ptr(), block_table.data_ptr(), block_table.stride(0),
            None if sm.group_start is None else sm.group_start.data_ptr(),
            None if sm.group_order is None else sm.group_order.data_ptr(), num_rows, num_groups,
            num_heads, head_dim, block_size, num_blocks, float(scale), _dtype_code(query.dtype),
            ctypes.byref(meta), _stream(dev),
        )
    )


def cache_pointer_table(caches: list[torch.Tensor]) -> torch.Tensor:
    """Device int64 tensor of cache base addresses, the ``caches`` argument of copy_blocks."""
    if not caches:
        raise ValueError("no caches")
    dev = _require_gpu(*caches)
    shape, dtype = caches[0].shape, caches[0].dtype
    for c in caches:
        if c.shape != shape or c.dtype != dtype or not c.is_contiguous():
            raise ValueError("caches must be contiguous tensors of one shape and dtype")
    return torch.tensor([c.data_ptr() for c in caches], dtype=torch.int64, device=dev)


def copy_blocks(
    caches: list[torch.Tensor],
    src: torch.Tensor,
    dst: torch.Tensor,
    pointer_table: torch.Tensor | None = None,
    staged: bool = False,
) -> None:
    """``cache[dst[p]] = cache[src[p]]`` for every cache and pair, in one launch.

    Counterpart of ModelRunner._copy_blocks (vflorence/engine/model_runner.py:162-167),
    which runs ``index_copy_(0, dst, index_select(0, src))`` per cache: every source is
    read before any destination is written.  The caller holds the pairs on the host
    and passes ``staged=copy_pairs_need_staging(pairs)``: when a destination block is
    also a source, the copy goes through a staging buffer to keep that order;
    otherwise it is a single direct pass.
    """
    if not caches:
        return
    dev = _require_gpu(*caches, src, dst)
    if src.dtype != torch.int64 or dst.dtype != torch.int64 or src.shape != dst.shape or src.dim() != 1:
        raise ValueError("src/dst must be int64 vectors of one length")
    if src.numel() == 0:
        return
    if pointer_table is None:
        pointer_table = cache_pointer_table(caches)
    elif pointer_table.dtype != torch.int64 or pointer_table.numel() != len(caches):
        raise ValueError("pointer_table must be int64 with one entry per cache")
    num_blocks = caches[0].shape[0]
    block_bytes = caches[0][0].numel() * caches[0].element_size()
    src = src.contiguous()
    dst = dst.contiguous()
    staging = None
    if staged:
        staging = torch.empty(len(caches) * src.numel() * block_bytes, dtype=torch.uint8, device=dev)
    check(
        lib.vfl_copy_blocks(
            pointer_table.data_ptr(), len(caches), src.data_ptr(), dst.data_ptr(), src.numel(),
            block_bytes, num_blocks, None if staging is None else staging.data_ptr(),
            _stream(dev),
        )
    )


class BlockCopier:
    """``copy_blocks`` over a fixed set of caches, checked once: the per-step call of a
    runner passes only the pair vectors (device int64, validated by the library's host
    checks against the pool size)."""

    def __init__(self, caches: list[torch.Tensor]):
        self.pointer_table = cache_pointer_table(caches)
        self._caches = list(caches)  # the table holds their addresses: keep them alive
        self.device = self.pointer_table.device
        self.num_caches = len(caches)
        self.num_blocks = caches[0].shape[0]
        self.block_bytes = caches[0][0].numel() * caches[0].element_size()

    def __call__(self, src: torch.Tensor, dst: torch.Tensor, staged: bool = False) -> None:
        n = src.numel()
        if (src.dtype != torch.int64 or dst.dtype != torch.int64 or dst.numel() != n
                or not src.is_contiguous() or not dst.is_contiguous()
                or src.device != self.device or dst.device != self.device):
            raise ValueError("src/dst must be contiguous int64 vectors of one length on the "
                             "caches' device")
        if n == 0:
            return
        staging = None
        if staged:
            staging = torch.empty(self.num_caches * n * self.block_bytes, dtype=torch.uint8,
                                  device=self.device)
        check(lib.vfl_copy_blocks(self.pointer_table.data_ptr(), self.num_caches,
                                  src.data_ptr(), dst.data_ptr(), n, self.block_bytes,
                                  self.num_blocks, None if staging is None else staging.data_ptr(),
                                  _stream(self.device)))


def copy_pairs_need_staging(pairs: list[tuple[int, int]]) -> bool:
    """True when a destination block is also a source block; raises on repeated dsts."""
    dsts = [d for _, d in pairs]
    if len(set(dsts)) != len(dsts):
        raise ValueError("copy-on-write pairs repeat a destination block")
    return not set(dsts).isdisjoint(s for s, _ in pairs)
