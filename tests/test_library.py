"""The C-ABI libraries load and export what their headers declare
(include/vflorence_amd.h: the GPU library; include/vfl_engine.h: the engine's host
core), and the GPU library's host-side planning and argument checks behave (no GPU
work is launched here)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "vflorence_amd.h")


HOST_HEADER = os.path.join(ROOT, "include", "vfl_engine.h")


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vfl_[a-z_0-9]+)\s*\(", text)))


def test_host_core_exports_every_declared_symbol():
    from vflorence_amd.engine import core

    declared = declared_functions(HOST_HEADER)
    assert declared and sorted(core.EXPORTED_SYMBOLS) == declared
    raw = ctypes.CDLL(core.LIB_PATH)
    for name in declared:
        assert hasattr(raw, name), name


def test_library_exports_every_declared_symbol():
    from vflorence_amd import _lib

    declared = declared_functions()
    assert declared, "no declarations found"
    assert sorted(_lib.EXPORTED_SYMBOLS) == declared
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared:
        assert hasattr(raw, name), name


def test_version_and_isa():
    from vflorence_amd import hip_attn
    from vflorence_amd._lib import lib

    assert lib.vfl_version() >= 100
    import torch

    assert hip_attn.get_isa(torch.bfloat16, 16, 64) == "gfx950"
    assert hip_attn.get_isa(torch.float32, 16, 128) == "gfx950"
    with pytest.raises(ValueError):
        hip_attn.get_isa(torch.bfloat16, 24, 64)
    # 32-token blocks: the reference's block size on x86 (vflorence/config.py:42)
    assert hip_attn.get_isa(torch.bfloat16, 32, 64) == "gfx950"
    assert hip_attn.get_isa(torch.float32, 32, 80) == "gfx950"
    with pytest.raises(ValueError):
        hip_attn.get_isa(torch.bfloat16, 16, 72)
    # the reference's head sizes (vflorence/layers/attention.py:6), every dtype
    for d in (32, 48, 64, 80, 96, 112, 128, 160, 192, 224, 256, 512):
        for dt in (torch.float32, torch.bfloat16, torch.float16):
            assert hip_attn.get_isa(dt, 16, d) == "gfx950", (dt, d)
        rc, m = plan(8, 8, 4, d, 20)
        assert rc == 0 and m.head_dim == d


def plan(rows, groups, heads, dim, max_blocks, gmax=1, nw=0, dtype=1, tables=0):
    from vflorence_amd._lib import SchedMeta, lib

    meta = SchedMeta()
    rc = lib.vfl_get_scheduler_metadata(rows, groups, heads, dim, 16, max_blocks, gmax, dtype, nw,
                                        tables, ctypes.byref(meta))
    return rc, meta


def test_scheduler_metadata_plan():
    rc, m = plan(256, 256, 16, 64, 64)
    assert rc == 0
    assert (m.num_rows, m.num_groups, m.num_heads, m.head_dim) == (256, 256, 16, 64)
    assert m.max_blocks_per_seq == 64 and m.max_group_size == 1
    assert m.waves_per_workgroup in (1, 2, 4, 8)
    # 256 ragged rows (4096 workgroups) and 64 x 4 beams (1024 workgroups): four
    assert m.waves_per_workgroup == 4
    rc, m = plan(256, 64, 16, 64, 64, gmax=4)
    assert rc == 0 and m.waves_per_workgroup == 4 and m.max_group_size == 4
    # few workgroups: more waves each
    rc, m = plan(8, 8, 16, 64, 64)
    assert rc == 0 and m.waves_per_workgroup == 8
    # never more waves than blocks in the longest context
    rc, m = plan(4, 4, 16, 64, 1)
    assert rc == 0 and m.waves_per_workgroup == 1
    rc, m = plan(8, 2, 12, 64, 40, gmax=4, nw=4)
    assert rc == 0 and m.waves_per_workgroup == 4


@pytest.mark.parametrize(
    "kwargs",
    [
        dict(gmax=9),  # beams per group above the compiled maximum
        dict(gmax=0),
        dict(dim=72),  # not one of the reference's head sizes: no kernel
        dict(dim=1024),
        dict(groups=300),  # more groups than rows
        dict(nw=3),  # not a power of two
        dict(nw=16),
        dict(tables=2),  # neither shared nor own tables
    ],
)
def test_scheduler_metadata_rejects(kwargs):
    args = dict(rows=256, groups=256, heads=16, dim=64, max_blocks=64)
    args.update(kwargs)
    rc, _ = plan(**args)
    assert rc != 0


def test_attention_validates_before_launch():
    """Bad calls return an error code and a message; nothing is enqueued."""
    from vflorence_amd._lib import lib

    rc, meta = plan(4, 4, 16, 64, 8, nw=4)
    assert rc == 0
    fake = ctypes.c_void_p(0x1000)

    def call(rows=4, groups=4, dim=64, stride=8, meta_=meta, q=fake, kc=fake, group_start=None):
        return lib.vfl_attention_with_kv_cache(q, 3072, 64, kc, fake, fake, fake, fake, stride,
                                               group_start, None, rows, groups, 16, dim, 16, 100,
                                               0.125, 1, ctypes.byref(meta_), None)

    # metadata made for other sizes
    assert call(rows=5, groups=5) == -1
    assert b"metadata" in lib.vfl_last_error()
    # table narrower than the plan
    assert call(stride=4) == -1
    # unsupported head size
    assert call(dim=72) == -2
    # grouped counts without a group table
    rc2, meta2 = plan(4, 2, 16, 64, 8)
    assert call(groups=2, meta_=meta2) == -1
    # null / misaligned pointers
    assert call(q=None) == -1
    assert call(kc=ctypes.c_void_p(0x1008)) == -1
    # zero rows is a no-op
    rc0, meta0 = plan(0, 0, 16, 64, 8)
    assert rc0 == 0
    assert lib.vfl_attention_with_kv_cache(None, 0, 0, None, None, None, None, None, 8, None, None,
                                           0, 0, 16, 64, 16, 100, 0.125, 1, ctypes.byref(meta0),
                                           None) == 0


def test_fused_self_attention_groups_need_own_tables():
    """Row groups in the fused KV-write entry point must come with metadata that says
    every row keeps its own block table; the call is refused before any launch."""
    from vflorence_amd._lib import VFL_GROUP_OWN_TABLES, lib

    fake = ctypes.c_void_p(0x1000)

    def call(tables):
        rc, meta = plan(4, 2, 16, 64, 8, gmax=2, tables=tables)
        assert rc == 0 and meta.group_tables == tables
        # num_rows 0: validation only, nothing is launched
        return lib.vfl_self_attention_with_kv_write(
            fake, 3072, 64, fake, 3072, 64, fake, 3072, 64, fake, fake, fake, fake, fake, fake,
            8, fake, None, 0, 0, 16, 64, 16, 100, 0.125, 1, ctypes.byref(meta), None)

    assert call(0) == -1
    assert b"VFL_GROUP_OWN_TABLES" in lib.vfl_last_error()
    assert call(VFL_GROUP_OWN_TABLES) == 0


def test_reshape_and_copy_validate_before_launch():
    from vflorence_amd._lib import lib

    # bad dtype / head_dim not a multiple of the 16-byte vector
    assert lib.vfl_reshape_and_cache(None, None, 0, 0, 0, 0, None, None, None, 4, 16, 64, 16, 10,
                                     7, None) == -1
    assert lib.vfl_reshape_and_cache(None, None, 0, 0, 0, 0, None, None, None, 4, 16, 60, 16, 10,
                                     1, None) == -2
    assert lib.vfl_reshape_and_cache(None, None, 0, 0, 0, 0, None, None, None, 0, 16, 64, 16, 10,
                                     1, None) == 0
    # block sizes without an attention kernel are refused before anything launches
    # (the 16-bit V layout would land outside the block-head slice)
    for bs in (8, 24, 18, 64):
        assert lib.vfl_reshape_and_cache(None, None, 0, 0, 0, 0, None, None, None, 4, 16, 64,
                                         bs, 10, 1, None) == -2
        assert b"block_size" in lib.vfl_last_error()
    assert lib.vfl_copy_blocks(None, 24, None, None, 5, 1000, 10, None, None) == -1  # not /16
    assert lib.vfl_copy_blocks(None, 24, None, None, 0, 1024, 10, None, None) == 0
    assert lib.vfl_copy_blocks(None, 24, None, None, 5, 1024, 10, None, None) == -1  # nulls
    # the no-allocation variant: the same checks, and staging beyond the library's
    # buffer refused on the host before anything launches
    from vflorence_amd._lib import NOALLOC_STAGING_BYTES

    assert lib.vfl_copy_blocks_noalloc(None, 24, None, None, 5, 1000, 10, 1, None) == -1
    assert lib.vfl_copy_blocks_noalloc(None, 24, None, None, 0, 1024, 10, 1, None) == 0
    assert lib.vfl_copy_blocks_noalloc(None, 24, None, None, 5, 1024, 10, 0, None) == -1
    fake = 1 << 20
    pairs = NOALLOC_STAGING_BYTES // (24 * 32768) + 1
    assert lib.vfl_copy_blocks_noalloc(fake, 24, fake, fake, pairs, 32768, 10, 1, None) == -1
    assert b"exceeds" in lib.vfl_last_error()


def test_linear_validates_before_launch():
    from vflorence_amd._lib import lib

    assert lib.vfl_linear_packed_elems(1000, 512) == 1024 * 512  # rows padded to 32
    assert lib.vfl_linear_packed_elems(0, 512) == 0

    def call(rows=4, out=1024, inp=1024, dtype=1, xs=1024, ys=1024, ptr=None, flags=0):
        return lib.vfl_linear(ptr, xs, ptr, None, ptr, ys, rows, out, inp, flags, dtype, None)

    assert call(dtype=0) == -2                  # fp32: no kernel
    assert call(inp=768 + 128) == -2            # in_features not a multiple of 256
    assert call(rows=65535 * 32 + 1) == -2
    assert call(rows=-1) == -1 and call(out=0) == -1
    assert call(xs=512) == -1 and call(ys=1000) == -1  # strides shorter than a row
    assert call(rows=0) == 0                    # nothing to do, nothing dereferenced
    assert call() == -1                         # null pointers
    assert b"null" in lib.vfl_last_error()
    assert call(ptr=16 * 1000 + 8) == -1        # 8-byte aligned x / weight
    assert b"aligned" in lib.vfl_last_error()
    assert call(flags=8) == -1                  # unknown flag
    assert call(out=1000, flags=4) == -2        # packed output needs out % 32 == 0
    assert call(xs=0, flags=2) == -1            # packed x: stride ignored, nulls caught
    assert b"null" in lib.vfl_last_error()

    def pack(out=1024, inp=1024, stride=1024, dtype=1, ptr=None):
        return lib.vfl_pack_linear_weight(ptr, stride, out, inp, ptr, dtype, None)

    assert pack(dtype=2 + 5) == -2 and pack(inp=300) == -2
    assert pack(stride=1000) == -1 and pack() == -1
    assert pack(ptr=16 * 1000 + 8) == -1


def test_embed_layer_norm_validates_before_launch():
    """vfl_embed_layer_norm refuses bad sizes, null or misaligned pointers and empty tables
    with an error code and message, before touching memory or the GPU."""
    from vflorence_amd._lib import lib

    a = 16 * 1000  # a 16-byte aligned stand-in address (never dereferenced)

    def call(ids=a, pos=a, rows=4, tok=a, tok_rows=50, pos_t=a, pos_rows=12, dim=64,
             stride=64, dtype=1, out=a):
        return lib.vfl_embed_layer_norm(ids, pos, rows, tok, tok_rows, stride, 1.0, pos_t,
                                        pos_rows, stride, 2, a, a, out, stride, dim, 1e-5,
                                        dtype, None)

    assert call(dtype=7) == -1 and b"dtype" in lib.vfl_last_error()
    assert call(dim=66) == -1 and call(dim=8192) == -1   # a multiple of 4, at most 4096
    assert call(stride=32) == -1                          # stride shorter than a row
    assert call(tok=a + 4) == -1 and b"aligned" in lib.vfl_last_error()  # 4 bf16 = 8 bytes
    assert call(out=None) == -1 and b"null" in lib.vfl_last_error()
    assert call(ids=None) == -1 and call(pos=None) == -1
    assert call(tok_rows=0) == -1 and call(pos_rows=0) == -1
    assert call(rows=0) == 0                              # nothing to do, nothing read


def test_cpu_tensors_are_rejected():
    import torch

    from vflorence_amd import hip_attn

    k = torch.zeros(4, 2, 16, 64, dtype=torch.bfloat16)
    x = torch.zeros(3, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="no CPU path"):
        hip_attn.reshape_and_cache(x, x, k, k, torch.zeros(3, dtype=torch.int64))
    # a pool of a block size with no kernel is refused on the host, whatever the device
    k24 = torch.zeros(4, 2, 24, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="block_size=24"):
        hip_attn.reshape_and_cache(x, x, k24, k24, torch.zeros(3, dtype=torch.int64))


def _header_struct_layout(tmp_path):
    """(field, offset) of the header's vfl_sched_meta and its size, as a C compiler lays
    it out (gcc on a tiny program that includes the header)."""
    import subprocess

    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    body = re.search(r"typedef struct vfl_sched_meta \{(.*?)\} vfl_sched_meta;", text, re.S)
    fields = re.findall(r"\b(\w+)\s*;", body.group(1))
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "vflorence_amd.h"\n'
                   "int main(void) {\n"
                   + "".join(f'  printf("{f} %zu\\n", offsetof(vfl_sched_meta, {f}));\n'
                             for f in fields)
                   + '  printf("sizeof %zu\\n", sizeof(vfl_sched_meta));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-x", "c", "-I", os.path.join(ROOT, "include"), str(src), "-o",
                    str(exe)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True,
                           text=True).stdout.split("\n")
    pairs = [ln.split() for ln in lines if ln]
    return [(n, int(o)) for n, o in pairs[:-1]], int(pairs[-1][1])


def _integration_sched_meta():
    """Execute the SchedMeta class of INTEGRATION.md's binding snippet (only that class
    and its size assertion) and return it."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = re.search(r"```python\n(.*?)```", text, re.S).group(1)
    start = block.index("class SchedMeta(")
    end = block.index("\n\n", start)
    snippet = block[start:end]
    scope = {"ctypes": ctypes}
    exec(snippet, scope)
    return scope["SchedMeta"], snippet


def test_sched_meta_bindings_match_the_header(tmp_path):
    """The scheduler-metadata struct has one layout everywhere a caller meets it: the
    header (compiled), the package's binding and the binding INTEGRATION.md shows a
    maintainer -- same field names in the same order, same offsets, 64 bytes.  A short
    copy would let vfl_get_scheduler_metadata write past the caller's struct."""
    from vflorence_amd import _lib

    c_fields, c_size = _header_struct_layout(tmp_path)
    assert c_size == 64
    for binding in (_lib.SchedMeta, _integration_sched_meta()[0]):
        names = [f for f, _ in binding._fields_]
        assert names == [f for f, _ in c_fields], binding
        assert [getattr(binding, f).offset for f in names] == [o for _, o in c_fields]
        assert ctypes.sizeof(binding) == c_size
    assert "sizeof(SchedMeta) == 64" in _integration_sched_meta()[1]
