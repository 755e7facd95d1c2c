"""ctypes binding of the engine's native host core (libvfl_host.so, include/vfl_engine.h).

``BlockPool`` is the paged KV block pool (reference counts, FIFO free list,
copy-on-write); ``EngineCore`` the decode loop's host state (waiting and running
hypotheses, admission, step metadata, greedy and beam-search updates).  Both are thin:
every call validates its arguments and forwards plain pointers and sizes.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(HERE, "libvfl_host.so")

OK, E_INVALID, E_FULL, E_STATE = 0, -1, -2, -3

_i32, _i64, _f64, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_double, ctypes.c_void_p
_pi32, _pi64 = ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int64)

_SIGNATURES = {
    "vfl_host_last_error": (ctypes.c_char_p, []),
    "vfl_pool_create": (_vp, [_i32, _i32]),
    "vfl_pool_destroy": (None, [_vp]),
    "vfl_pool_reset": (None, [_vp]),
    "vfl_pool_num_blocks": (_i32, [_vp]),
    "vfl_pool_num_free": (_i32, [_vp]),
    "vfl_pool_refcounts": (None, [_vp, _vp]),
    "vfl_pool_free_list": (None, [_vp, _vp]),
    "vfl_pool_prepare_write": (ctypes.c_int, [_vp, _vp, _i32, _i32, _pi32, _pi32]),
    "vfl_pool_blocks_needed": (_i64, [_vp, _vp, _i32]),
    "vfl_pool_share": (ctypes.c_int, [_vp, _vp, _i32]),
    "vfl_pool_release": (ctypes.c_int, [_vp, _vp, _i32]),
    "vfl_engine_create": (_vp, [_i32, _i32, _i32]),
    "vfl_engine_destroy": (None, [_vp]),
    "vfl_engine_pool": (_vp, [_vp]),
    "vfl_engine_reset": (None, [_vp]),
    "vfl_engine_add_request": (ctypes.c_int, [_vp, _i64, _vp, _i32, _i32, _i32, _vp, _i32, _f64,
                                              _i32]),
    "vfl_engine_num_waiting": (_i32, [_vp]),
    "vfl_engine_num_running": (_i32, [_vp]),
    "vfl_engine_num_pending_beams": (_i32, [_vp]),
    "vfl_engine_schedule": (ctypes.c_int, [_vp, _vp, _i32, _pi32, _pi32, _pi32]),
    "vfl_engine_pack": (ctypes.c_int, [_vp, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                       _vp, _vp, _vp, _vp, _pi32]),
    "vfl_engine_max_table_len": (_i32, [_vp]),
    "vfl_engine_max_row_tokens": (_i32, [_vp]),
    "vfl_engine_history": (ctypes.c_int, [_vp, _vp, _i32]),
    "vfl_engine_greedy_update": (ctypes.c_int, [_vp, _vp, _i32]),
    "vfl_engine_beam_update": (ctypes.c_int, [_vp, _vp, _vp, _i32, _i32]),
    "vfl_engine_abort_request": (ctypes.c_int, [_vp, _i64]),
    "vfl_engine_next_finished": (ctypes.c_int, [_vp, _pi64, _vp, _i32, _pi32]),
    "vfl_engine_row": (ctypes.c_int, [_vp, _i32, _pi64, _pi32, _pi32, ctypes.POINTER(_f64), _pi32,
                                      _vp, _vp, _i32]),
}
EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; "
                          "g.build()'` (g++). The engine has no other host core.")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


lib = _load()


def _check(status: int) -> int:
    if status < 0:
        msg = lib.vfl_host_last_error().decode(errors="replace")
        if status == E_FULL:
            raise RuntimeError(msg)
        if status == E_INVALID:
            raise ValueError(msg)
        raise RuntimeError(msg)
    return status


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


class BlockPool:
    """The paged KV block pool (``vfl_pool``); ``owner`` keeps a borrowed pool's engine
    alive."""

    def __init__(self, num_blocks: int = 0, block_size: int = 16, *, handle=None, owner=None):
        if handle is None:
            handle = lib.vfl_pool_create(num_blocks, block_size)
            if not handle:
                raise ValueError(lib.vfl_host_last_error().decode())
            self._owned = True
        else:
            self._owned = False
        self._h, self._owner = handle, owner
        self.block_size = block_size

    def __del__(self):
        if getattr(self, "_owned", False) and self._h:
            lib.vfl_pool_destroy(self._h)
            self._h = None

    @property
    def num_blocks(self) -> int:
        return lib.vfl_pool_num_blocks(self._h)

    @property
    def num_free(self) -> int:
        return lib.vfl_pool_num_free(self._h)

    def refcounts(self) -> np.ndarray:
        out = np.empty(self.num_blocks, dtype=np.int32)
        lib.vfl_pool_refcounts(self._h, _ptr(out))
        return out

    def free_list(self) -> np.ndarray:
        out = np.empty(self.num_free, dtype=np.int32)
        lib.vfl_pool_free_list(self._h, _ptr(out))
        return out

    def reset(self) -> None:
        lib.vfl_pool_reset(self._h)

    def prepare_write(self, table: list[int], cached: int) -> tuple[int, int, int]:
        """(action, block, src) of ``vfl_pool_prepare_write``."""
        arr = np.asarray(table, dtype=np.int32)
        block, src = ctypes.c_int32(-1), ctypes.c_int32(-1)
        action = _check(lib.vfl_pool_prepare_write(self._h, _ptr(arr), len(arr), cached,
                                                   ctypes.byref(block), ctypes.byref(src)))
        return action, block.value, src.value

    def blocks_needed(self, write_blocks) -> int:
        arr = np.asarray(write_blocks, dtype=np.int32)
        return _check(lib.vfl_pool_blocks_needed(self._h, _ptr(arr), len(arr)))

    def share(self, table: list[int]) -> None:
        arr = np.asarray(table, dtype=np.int32)
        _check(lib.vfl_pool_share(self._h, _ptr(arr), len(arr)))

    def release(self, table: list[int]) -> None:
        arr = np.asarray(table, dtype=np.int32)
        _check(lib.vfl_pool_release(self._h, _ptr(arr), len(arr)))


class RowView:
    """A snapshot of one running hypothesis of an ``EngineCore``."""

    __slots__ = ("request_id", "token_ids", "block_table", "num_cached_tokens", "cum_logprob")

    def __init__(self, request_id, token_ids, block_table, num_cached_tokens, cum_logprob):
        self.request_id = request_id
        self.token_ids = token_ids
        self.block_table = block_table
        self.num_cached_tokens = num_cached_tokens
        self.cum_logprob = cum_logprob

    def __repr__(self) -> str:
        return (f"RowView(request_id={self.request_id}, tokens={self.token_ids}, "
                f"table={self.block_table}, cached={self.num_cached_tokens})")


_PACK_I32 = ("context_lens", "order", "group_start", "tables")
_PACK_NAMES = ("input_ids", "positions", "slots", "lengths", "copy_src", "copy_dst",
               "context_lens", "order", "group_start", "tables", "row_requests")


class EngineCore:
    """The decode loop's host state (``vfl_engine``)."""

    def __init__(self, num_blocks: int, block_size: int, max_num_seqs: int):
        self._h = lib.vfl_engine_create(num_blocks, block_size, max_num_seqs)
        if not self._h:
            raise ValueError(lib.vfl_host_last_error().decode())
        self.block_size, self.max_num_seqs = block_size, max_num_seqs
        self.pool = BlockPool(block_size=block_size, handle=lib.vfl_engine_pool(self._h),
                              owner=self)
        self._admitted = np.empty(max(1, max_num_seqs), dtype=np.int64)
        self._n = [ctypes.c_int32() for _ in range(4)]
        self._pack_ptrs = {}  # id(views) -> (views, arrays, addresses, rows, tables shape)
        self._out_id = ctypes.c_int64()
        self._out_tokens = np.empty(1024, dtype=np.int32)
        self.num_rows = self.num_pairs = 0

    def __del__(self):
        if getattr(self, "_h", None):
            lib.vfl_engine_destroy(self._h)
            self._h = None

    def reset(self) -> None:
        lib.vfl_engine_reset(self._h)
        self.num_rows = self.num_pairs = 0

    def add_request(self, request_id: int, prompt: list[int], num_beams: int, max_tokens: int,
                    eos: list[int], length_penalty: float, early_stopping: bool) -> None:
        p = np.asarray(prompt, dtype=np.int32)
        e = np.asarray(sorted(eos), dtype=np.int32)
        _check(lib.vfl_engine_add_request(self._h, request_id, _ptr(p), len(p), num_beams,
                                          max_tokens, _ptr(e), len(e), float(length_penalty),
                                          int(bool(early_stopping))))
        self._out_tokens = np.empty(max(self._out_tokens.size, max_tokens + 1), dtype=np.int32)

    @property
    def num_waiting(self) -> int:
        return lib.vfl_engine_num_waiting(self._h)

    @property
    def num_running(self) -> int:
        return lib.vfl_engine_num_running(self._h)

    @property
    def num_pending_beams(self) -> int:
        return lib.vfl_engine_num_pending_beams(self._h)

    def schedule(self) -> list[int]:
        """Admission + capacity for a step; returns the admitted request ids and sets
        ``num_rows`` / ``num_pairs``.  RuntimeError when the pool cannot cover it."""
        na, nr, npairs = self._n[:3]
        _check(lib.vfl_engine_schedule(self._h, _ptr(self._admitted), self._admitted.size,
                                       ctypes.byref(na), ctypes.byref(nr), ctypes.byref(npairs)))
        self.num_rows, self.num_pairs = nr.value, npairs.value
        return self._admitted[: na.value].tolist()

    def pack(self, padded: int, table_width: int, max_group: int, views: dict) -> bool:
        """The step's metadata into the numpy ``views`` (int64 input_ids, positions,
        slots, lengths, copy_src, copy_dst, row_requests; int32 context_lens, order,
        group_start, tables [rows, table_width]); returns whether the rows form beam
        groups."""
        grouped = self._n[3]
        ptrs = self._pack_ptrs.get(id(views))
        # addresses of a views dict's arrays, taken once and kept with the arrays they
        # belong to (an array replaced under its name is seen and re-read)
        if (ptrs is None or ptrs[0] is not views
                or any(views[k] is not a for k, a in zip(_PACK_NAMES, ptrs[1]))):
            arrays = tuple(views[k] for k in _PACK_NAMES)
            for k, a in zip(_PACK_NAMES, arrays):
                want = np.int32 if k in _PACK_I32 else np.int64
                if a.dtype != want or not a.flags.c_contiguous:
                    raise ValueError(f"pack: {k} must be a contiguous {want.__name__} array")
            ptrs = (views, arrays, [a.ctypes.data for a in arrays],
                    min(len(views[k]) for k in _PACK_NAMES if k not in ("tables", "group_start")),
                    views["tables"].shape)
            self._pack_ptrs = {id(views): ptrs}
        cap, tshape = ptrs[3], ptrs[4]
        if (padded > cap or padded >= len(views["group_start"]) or len(tshape) != 2
                or tshape[0] < padded or tshape[1] != table_width):
            raise ValueError(f"pack: {padded} rows of width {table_width} do not fit the views "
                             f"(rows {cap}, tables {tuple(tshape)})")
        _check(lib.vfl_engine_pack(self._h, padded, table_width, max_group, *ptrs[2],
                                   ctypes.byref(grouped)))
        return bool(grouped.value)

    def max_table_len(self) -> int:
        return lib.vfl_engine_max_table_len(self._h)

    def history(self) -> np.ndarray:
        """[rows, longest] token histories, left-padded with -1."""
        width = max(1, lib.vfl_engine_max_row_tokens(self._h))
        out = np.empty((self.num_running, width), dtype=np.int64)
        _check(lib.vfl_engine_history(self._h, _ptr(out), width))
        return out

    def greedy_update(self, tokens: np.ndarray) -> None:
        t = np.ascontiguousarray(tokens, dtype=np.int64)
        _check(lib.vfl_engine_greedy_update(self._h, _ptr(t), len(t)))

    def beam_update(self, scores: np.ndarray, ids: np.ndarray) -> None:
        s = np.ascontiguousarray(scores, dtype=np.float32)
        i = np.ascontiguousarray(ids, dtype=np.int64)
        if s.shape != i.shape or s.ndim != 2:
            raise ValueError("scores and ids must be [rows, k] of one shape")
        _check(lib.vfl_engine_beam_update(self._h, _ptr(s), _ptr(i), s.shape[0], s.shape[1]))

    def abort_request(self, request_id: int) -> bool:
        """Drop a request between steps; False if it was not known."""
        return bool(_check(lib.vfl_engine_abort_request(self._h, request_id)))

    def finished(self) -> list[tuple[int, list[int]]]:
        """Requests that ended since the last call: (request id, completion tokens)."""
        out = []
        n = self._n[0]
        while True:
            st = _check(lib.vfl_engine_next_finished(self._h, ctypes.byref(self._out_id),
                                                     _ptr(self._out_tokens),
                                                     self._out_tokens.size, ctypes.byref(n)))
            if st == 0:
                return out
            out.append((self._out_id.value, self._out_tokens[: n.value].tolist()))

    def row(self, r: int) -> RowView:
        rid, nt, cached, tl = ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        cum = ctypes.c_double()
        _check(lib.vfl_engine_row(self._h, r, ctypes.byref(rid), ctypes.byref(nt),
                                  ctypes.byref(cached), ctypes.byref(cum), ctypes.byref(tl), None,
                                  None, 0))
        cap = max(nt.value, tl.value, 1)
        tokens, table = np.empty(cap, np.int32), np.empty(cap, np.int32)
        _check(lib.vfl_engine_row(self._h, r, None, None, None, None, None, _ptr(tokens),
                                  _ptr(table), cap))
        return RowView(rid.value, tokens[: nt.value].tolist(), table[: tl.value].tolist(),
                       cached.value, cum.value)

    def rows(self) -> list[RowView]:
        return [self.row(r) for r in range(self.num_running)]
