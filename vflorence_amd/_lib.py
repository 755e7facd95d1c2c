"""ctypes binding of libvflorence_amd.so, the C ABI declared in include/vflorence_amd.h.

The library is built in-tree by ``vflorence_amd._build.build_library()`` (hipcc,
``--offload-arch=gfx950``).  There is no other implementation of these entry points:
importing this module without the built library raises, so nothing can silently
run a fallback.
"""

from __future__ import annotations

import ctypes
import os

LIB_NAME = "libvflorence_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

VFL_FLOAT32, VFL_BFLOAT16, VFL_FLOAT16 = 0, 1, 2
VFL_GROUP_SHARED_TABLE, VFL_GROUP_OWN_TABLES = 0, 1
VFL_OK = 0

# Every symbol include/vflorence_amd.h declares; tests check the library exports them.
EXPORTED_SYMBOLS = (
    "vfl_last_error",
    "vfl_version",
    "vfl_get_isa",
    "vfl_reshape_and_cache",
    "vfl_get_scheduler_metadata",
    "vfl_group_plan_stride",
    "vfl_build_group_plan",
    "vfl_fold_plan_copies",
    "vfl_slot_descriptor_stride",
    "vfl_build_slot_descriptors",
    "vfl_attention_with_kv_cache",
    "vfl_self_attention_with_kv_write",
    "vfl_copy_blocks",
    "vfl_copy_blocks_noalloc",
    "vfl_add_layer_norm",
    "vfl_embed_layer_norm",
    "vfl_logprob_topk",
    "vfl_linear_packed_elems",
    "vfl_pack_linear_weight",
    "vfl_linear",
    "vfl_linear_residual",
    "vfl_linear_norm",
    "vfl_layer_norm_apply",
)


class SchedMeta(ctypes.Structure):
    """Mirror of ``struct vfl_sched_meta``."""

    _fields_ = [
        ("num_rows", ctypes.c_int64),
        ("num_groups", ctypes.c_int64),
        ("num_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("max_blocks_per_seq", ctypes.c_int32),
        ("waves_per_workgroup", ctypes.c_int32),
        ("max_group_size", ctypes.c_int32),
        ("group_tables", ctypes.c_int32),
        ("group_plan", ctypes.c_void_p),
        ("group_plan_stride", ctypes.c_int64),
        ("group_plan_slots", ctypes.c_int64),
    ]


_i64, _i32, _vp, _f32 = ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_float

_SIGNATURES = {
    "vfl_last_error": (ctypes.c_char_p, []),
    "vfl_version": (ctypes.c_int, []),
    "vfl_get_isa": (ctypes.c_char_p, [_i32, _i32, _i32]),
    "vfl_reshape_and_cache": (
        ctypes.c_int,
        [_vp, _vp, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _i64, _i32,
         _vp],
    ),
    "vfl_get_scheduler_metadata": (
        ctypes.c_int,
        [_i64, _i64, _i32, _i32, _i32, _i64, _i32, _i32, _i32, _i32, ctypes.POINTER(SchedMeta)],
    ),
    "vfl_group_plan_stride": (_i64, [_i32, _i64]),
    "vfl_fold_plan_copies": (ctypes.c_int, [_vp, _i64, _i64, _vp, _vp, _i64, _i64]),
    "vfl_slot_descriptor_stride": (_i64, [_i64]),
    "vfl_build_slot_descriptors": (
        ctypes.c_int, [_vp, _i64, _i32, _vp, _i64, _vp, _vp, _i64, _vp, _i64, _i64]),
    "vfl_build_group_plan": (
        ctypes.c_int,
        [_vp, _i64, _i32, _vp, _i64, _vp, _vp, _i64, _i32, _i64, _vp, _i64, _i64],
    ),
    "vfl_attention_with_kv_cache": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64, _i32, _i32, _i32,
         _i64, _f32, _i32, ctypes.POINTER(SchedMeta), _vp],
    ),
    "vfl_self_attention_with_kv_write": (
        ctypes.c_int,
        [_vp, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
         _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i64, _f32, _i32, ctypes.POINTER(SchedMeta),
         _vp],
    ),
    "vfl_copy_blocks": (
        ctypes.c_int,
        [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _vp, _vp],
    ),
    "vfl_copy_blocks_noalloc": (
        ctypes.c_int,
        [_vp, _i32, _vp, _vp, _i64, _i64, _i64, _i32, _vp],
    ),
    "vfl_add_layer_norm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i32, _f32, _i32, _vp],
    ),
    "vfl_embed_layer_norm": (
        ctypes.c_int,
        [_vp, _vp, _i64, _vp, _i64, _i64, _f32, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _i64, _i32,
         _f32, _i32, _vp],
    ),
    "vfl_logprob_topk": (
        ctypes.c_int,
        [_vp, _i64, _i64, _i32, _i32, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
         _i32, _i32, _vp, _vp, _vp],
    ),
    "vfl_linear_packed_elems": (ctypes.c_int64, [_i32, _i32]),
    "vfl_pack_linear_weight": (ctypes.c_int, [_vp, _i64, _i32, _i32, _vp, _i32, _vp]),
    "vfl_linear": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp],
    ),
    "vfl_linear_residual": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _f32, _vp, _i64, _vp, _i64, _i32, _i32,
         _i32, _i32, _vp],
    ),
    "vfl_linear_norm": (
        ctypes.c_int,
        [_vp, _i64, _vp, _f32, _vp, _vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp],
    ),
    "vfl_layer_norm_apply": (
        ctypes.c_int,
        [_vp, _i64, _vp, _vp, _vp, _f32, _vp, _i64, _i64, _i32, _i32, _vp],
    ),
}


# bytes of the library's per-GPU staging buffer (VFL_NOALLOC_STAGING_BYTES)
NOALLOC_STAGING_BYTES = 64 << 20


class LibraryMissing(ImportError):
    pass


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950). There is no fallback implementation."
        )
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = _load()


class HipAttnError(RuntimeError):
    """A C-ABI call returned an error status (the library's TORCH_CHECK equivalent)."""


def check(status: int) -> None:
    if status != VFL_OK:
        msg = lib.vfl_last_error().decode(errors="replace")
        raise HipAttnError(f"vflorence_amd error {status}: {msg}")
