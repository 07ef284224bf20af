"""Node-wide KV block manager on the native bookkeeping (``aegkv_bm_*``).

:class:`BlockManager` keeps the method names, arguments and errors of the
reference's ``BlockManager`` (aegaeon/aegaeon/block_manager.py:165-874) and
hands out the same block ids in the same order.  The bookkeeping — GPU FIFO
free lists, the CPU slab pool, block tables and pending moves — lives in
``libaegkv.so``; this class keeps what is asynchronous or Python-side in the
reference: the per-engine swap callables, the move events' completion handles,
``latest_events`` and the zombie list.

Where the reference awaits pending moves before reclaiming their source blocks
(_reclaim_blocks, block_manager.py:360-408), the library calls back into
:meth:`_wait_moves`, which waits on each pending move's handles (HIP events,
objects with ``synchronize()``, or callables) unless one of its requests has
finished (block_manager.py:373-376).
"""
from __future__ import annotations

import ctypes
import logging
import math
from dataclasses import dataclass
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _lib

logger = logging.getLogger(__name__)

BLOCK_LOCATION_CPU = -1  # block_manager.py:96
BLOCK_SIZE = 16          # aegaeon/aegaeon/config.py:13
_NO_SPACE = -9
_IN_USE = -10


def is_gpu(location: int) -> bool:
    return location >= 0


@dataclass
class BlockTable:  # block_manager.py:103-111 (a snapshot: edits do not flow back)
    location: int
    block_shape: Tuple[int, ...]
    blocks: List[int]


@dataclass(eq=False)
class MoveEvent:  # block_manager.py:114-131
    serial: int
    requests: List[Any]
    block_shape: Tuple[int, ...]
    source_location: int
    target_location: int
    source_blocks: List[int]
    event_handle_refs: Any = None


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int64)


def _ptr(a: np.ndarray):
    return a.ctypes.data if a.size else None


def _requests_of(batch) -> Sequence[Any]:
    return batch.requests if hasattr(batch, "requests") else batch


def _wait_handle(h) -> None:
    if h is None:
        return
    if isinstance(h, (list, tuple)):
        for x in h:
            _wait_handle(x)
    elif hasattr(h, "synchronize"):
        h.synchronize()
    elif callable(h):
        h()
    else:
        raise TypeError(f"cannot wait on move handle {h!r}")


class BlockManager:
    """Drop-in for the reference's ``BlockManager`` (block_manager.py:165)."""

    def __init__(self, cpu_num_slabs: int, cpu_slab_size_bytes: int, dtype_size: int = 2,
                 wait_move: Optional[Callable[[MoveEvent], None]] = None):
        self.block_size = BLOCK_SIZE
        self.dtype_size = dtype_size
        self.cpu_num_slabs = cpu_num_slabs
        self.cpu_slab_size_bytes = cpu_slab_size_bytes
        self._lib = _lib.load()
        self._wait_move = wait_move
        self._wait_error: Optional[BaseException] = None
        self._cb = _lib.BM_WAIT_FN(self._wait_moves)  # kept alive with the manager
        self._h = None
        self._create()

    def _create(self) -> None:
        h = ctypes.c_void_p()
        _lib.check(self._lib.aegkv_bm_create(self.cpu_num_slabs, self.cpu_slab_size_bytes,
                                             ctypes.byref(h)), "BlockManager")
        self._h = h.value
        _lib.check(self._lib.aegkv_bm_set_wait(self._h, ctypes.cast(self._cb, ctypes.c_void_p),
                                               None), "BlockManager")
        self._shape_ids: Dict[Tuple[int, ...], int] = {}
        self._shapes: List[Tuple[int, ...]] = []
        self.gpu_block_shape: Dict[int, Tuple[int, ...]] = {}
        self.gpu_num_max_blocks: Dict[int, int] = {}
        self.remote_callables: Dict[int, Callable] = {}
        self._moves: Dict[int, MoveEvent] = {}
        self.latest_events: Dict[int, Any] = {}
        self.zombie_request_ids: List[int] = []

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.aegkv_bm_destroy(h)

    def reset(self) -> None:  # block_manager.py:274-298
        self._lib.aegkv_bm_destroy(self._h)
        self._h = None
        self._create()

    # -- shapes ---------------------------------------------------------------
    def _get_block_size_bytes(self, block_shape) -> int:  # :239-240
        return math.prod(block_shape) * self.dtype_size

    def _shape_id(self, block_shape) -> int:
        shape = tuple(int(x) for x in block_shape)
        sid = self._shape_ids.get(shape)
        if sid is None:
            sid = len(self._shapes)
            _lib.check(self._lib.aegkv_bm_define_shape(self._h, sid,
                                                       self._get_block_size_bytes(shape)),
                       "define_shape")
            self._shape_ids[shape] = sid
            self._shapes.append(shape)
        return sid

    # -- reclaim callback -----------------------------------------------------
    def _wait_moves(self, _ctx, location: int, shape_id: int, serial: int) -> int:
        """Wait for every pending move out of ``location`` (CPU: of the shape)
        with a serial <= ``serial``; 0 lets the library reclaim them."""
        try:
            shape = self._shapes[shape_id] if 0 <= shape_id < len(self._shapes) else None
            done = [s for s, ev in self._moves.items()
                    if s <= serial and ev.source_location == location
                    and (is_gpu(location) or ev.block_shape == shape)]
            for s in sorted(done):
                ev = self._moves[s]
                if not any(getattr(r, "is_finished", False) for r in ev.requests):
                    if self._wait_move is not None:
                        self._wait_move(ev)
                    else:
                        _wait_handle(ev.event_handle_refs)
            for s in done:
                del self._moves[s]
            return 0
        except BaseException as e:  # no exception may cross the C ABI
            self._wait_error = e
            return 1

    def _check(self, rc: int, op: str, msg: str = "") -> None:
        if rc == 0:
            return
        err, self._wait_error = self._wait_error, None
        if err is not None:
            raise err
        if rc == _NO_SPACE:
            raise ResourceWarning(msg or f"{op}: not enough free blocks")
        if rc == _IN_USE:
            raise ValueError(msg or f"{op}: {_lib.strerror(rc)}")
        _lib.check(rc, op)

    # -- GPU spaces (:300-348, :600-602) ---------------------------------------
    def register_gpu_space(self, engine_id: int, num_max_blocks: int, block_shape,
                           remote_callable: Optional[Callable] = None) -> None:
        sid = self._shape_id(block_shape)
        rc = self._lib.aegkv_bm_register_gpu_space(self._h, engine_id, num_max_blocks, sid)
        self._check(rc, "register_gpu_space",
                    f"Error registering new GPU cache space for engine_id {engine_id}; "
                    "a request still resides in the cache.")
        # the library dropped this engine's pending moves and reclaimed CPU moves into it
        for s in [s for s, ev in self._moves.items()
                  if ev.source_location == engine_id or
                  (not is_gpu(ev.source_location) and ev.target_location == engine_id)]:
            del self._moves[s]
        self.gpu_block_shape[engine_id] = tuple(block_shape)
        self.gpu_num_max_blocks[engine_id] = num_max_blocks
        self.remote_callables[engine_id] = remote_callable

    def get_gpu_num_max_blocks(self, engine_id: int) -> int:
        assert engine_id in self.gpu_num_max_blocks, f"unknown gpu location {engine_id}"
        return self.gpu_num_max_blocks[engine_id]

    # -- allocation (:604-711) -------------------------------------------------
    def get_num_blocks_needed(self, request) -> int:
        return (request.get_input_len() + request.get_output_len() + self.block_size - 1
                ) // self.block_size

    def get_num_append_blocks_needed(self, request) -> int:
        bt = self.get_block_table(request.request_id)
        assert is_gpu(bt.location), f"request {request.request_id} is not on GPU"
        return self.get_num_blocks_needed(request) - len(bt.blocks)

    def allocate_blocks_by_count(self, request_ids: Sequence[int], num_blocks_needed: Sequence[int],
                                 engine_id: int) -> None:
        """allocate_blocks_batched with the totals already computed."""
        ids, need = _i64(request_ids), _i64(num_blocks_needed)
        if ids.shape != need.shape:
            raise ValueError("one count per request")
        rc = self._lib.aegkv_bm_allocate(self._h, engine_id, _ptr(ids), _ptr(need), ids.size)
        self._check(rc, "allocate_blocks_batched",
                    "request is allocated elsewhere; migrate it before allocating more blocks"
                    if rc == _IN_USE else "")

    async def allocate_blocks_batched(self, batched_requests, engine_id: int) -> None:
        reqs = _requests_of(batched_requests)
        if len(reqs) == 0:
            return
        self.allocate_blocks_by_count([r.request_id for r in reqs],
                                      [self.get_num_blocks_needed(r) for r in reqs], engine_id)

    def free_blocks(self, request_id: int) -> None:
        rc = self._lib.aegkv_bm_free(self._h, request_id)
        if rc == -2:
            raise AssertionError(f"request {request_id} not allocated")
        self._check(rc, "free_blocks")
        self.latest_events.pop(request_id, None)
        self.zombie_request_ids.append(request_id)

    def free_blocks_batched(self, requests) -> None:
        for r in requests:
            self.free_blocks(r.request_id)

    # -- tables ----------------------------------------------------------------
    def get_block_table(self, request_id: int) -> BlockTable:
        loc, sid, n = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int64()
        rc = self._lib.aegkv_bm_table(self._h, request_id, ctypes.byref(loc), ctypes.byref(sid),
                                      ctypes.byref(n), None, 0)
        if rc == -2:
            raise AssertionError(f"request {request_id} not allocated")
        self._check(rc, "get_block_table")
        out = np.empty(n.value, dtype=np.int64)
        self._check(self._lib.aegkv_bm_table(self._h, request_id, ctypes.byref(loc),
                                             ctypes.byref(sid), ctypes.byref(n), _ptr(out),
                                             out.size), "get_block_table")
        return BlockTable(loc.value, self._shapes[sid.value], out.tolist())

    def flat_block_tables(self, request_ids: Sequence[int]) -> Tuple[np.ndarray, np.ndarray]:
        """(offsets int64 [n + 1], ids int32) of the requests' tables, the
        layout ``aegkv_prepare_inputs`` takes."""
        ids = _i64(request_ids)
        offsets = np.empty(ids.size + 1, dtype=np.int64)
        self._check(self._lib.aegkv_bm_flat_tables(self._h, _ptr(ids), ids.size,
                                                   offsets.ctypes.data, None, 0), "flat_tables")
        flat = np.empty(int(offsets[-1]), dtype=np.int32)
        self._check(self._lib.aegkv_bm_flat_tables(self._h, _ptr(ids), ids.size,
                                                   offsets.ctypes.data, _ptr(flat), flat.size),
                    "flat_tables")
        return offsets, flat

    def is_all_requests_on_gpu(self, requests) -> bool:
        return all(is_gpu(self.get_block_table(r.request_id).location)
                   for r in _requests_of(requests))

    # -- moves (:778-874) --------------------------------------------------------
    def move_request_ids(self, request_ids: Sequence[int], target_location: int):
        """The bookkeeping half of move_requests: returns ``None`` when nothing
        moves, else ``(serial, moved_request_ids, source_block_ids,
        target_block_ids, is_swap_in, engine_id)`` for the swap call."""
        ids = _i64(request_ids)
        serial, nb = ctypes.c_int64(), ctypes.c_int64()
        swap_in, engine = ctypes.c_int32(), ctypes.c_int32()
        rc = self._lib.aegkv_bm_move(self._h, _ptr(ids), ids.size, target_location,
                                     ctypes.byref(serial), ctypes.byref(nb),
                                     ctypes.byref(swap_in), ctypes.byref(engine))
        if rc == -6:
            raise NotImplementedError("Migration is not implemented")
        if rc == -2:
            raise AssertionError("request not allocated")
        self._check(rc, "move_requests")
        if serial.value < 0:
            return None
        src = np.empty(nb.value, dtype=np.int64)
        dst = np.empty(nb.value, dtype=np.int64)
        moved = np.empty(ids.size, dtype=np.int64)
        n_moved = ctypes.c_int64()
        self._check(self._lib.aegkv_bm_move_ids(self._h, _ptr(src), _ptr(dst), src.size,
                                                _ptr(moved), moved.size, ctypes.byref(n_moved)),
                    "move_requests")
        return (serial.value, moved[:n_moved.value].tolist(), src.tolist(), dst.tolist(),
                bool(swap_in.value), engine.value)

    async def move_requests(self, requests, target_location: int) -> bool:
        reqs = list(_requests_of(requests))
        res = self.move_request_ids([r.request_id for r in reqs], target_location)
        if res is None:
            return False
        serial, moved_ids, src, dst, is_swap_in, engine = res
        by_id = {r.request_id: r for r in reqs}
        swapped = [by_id[rid] for rid in moved_ids]
        # the GPU side of a swap is its engine; the blocks have that engine's shape
        source_location = BLOCK_LOCATION_CPU if is_swap_in else engine
        source_event_handles = [self.latest_events.get(r.request_id) for r in swapped]
        remote = self.remote_callables.get(engine)
        event_refs = None
        if remote is not None:
            event_refs = remote("swap_blocks", moved_ids, src, dst, source_event_handles,
                                is_swap_in)
        self._moves[serial] = MoveEvent(serial, swapped, self.gpu_block_shape[engine],
                                        source_location, target_location, src, event_refs)
        for r in swapped:
            self.latest_events[r.request_id] = event_refs
        return True

    def complete_moves(self, location: int, block_shape=None, up_to_serial: Optional[int] = None):
        """Reclaim the moves out of ``location`` whose copies are known done."""
        sid = self._shape_id(block_shape) if block_shape is not None else 0
        last = max(self._moves, default=-1) if up_to_serial is None else up_to_serial
        self._check(self._lib.aegkv_bm_complete_moves(self._h, location, sid, last),
                    "complete_moves")
        for s in [s for s, ev in self._moves.items()
                  if s <= last and ev.source_location == location
                  and (is_gpu(location) or ev.block_shape == tuple(block_shape))]:
            del self._moves[s]

    # -- usage (:730-768) ----------------------------------------------------------
    def stats(self, location: int, block_shape=None) -> Tuple[int, int, int, int]:
        """(free, moving, slabs, used) blocks of an engine or a CPU shape."""
        sid = self._shape_ids.get(tuple(block_shape), -2) if block_shape is not None else 0
        vals = [ctypes.c_int64() for _ in range(4)]
        self._check(self._lib.aegkv_bm_stats(self._h, location, sid,
                                             *[ctypes.byref(v) for v in vals]), "stats")
        return tuple(v.value for v in vals)

    def free_list(self, location: int, block_shape=None) -> List[int]:
        sid = self._shape_ids.get(tuple(block_shape), -2) if block_shape is not None else 0
        n = ctypes.c_int64()
        self._check(self._lib.aegkv_bm_free_list(self._h, location, sid, None, 0,
                                                 ctypes.byref(n)), "free_list")
        out = np.empty(n.value, dtype=np.int64)
        self._check(self._lib.aegkv_bm_free_list(self._h, location, sid, _ptr(out), out.size,
                                                 ctypes.byref(n)), "free_list")
        return out.tolist()

    def log_block_usage(self) -> None:
        lines = ["---------- Block Usage ----------"]
        for engine_id, num_max in self.gpu_num_max_blocks.items():
            free, moving, _, _ = self.stats(engine_id)
            lines.append(f"[gpu (engine {engine_id})] {free} / {num_max} "
                         f"({free / max(num_max, 1) * 100:.2f}%) free; {moving} / {num_max} "
                         f"({moving / max(num_max, 1) * 100:.2f}%) moving; ")
        for shape in self._shapes:
            free, moving, slabs, used = self.stats(BLOCK_LOCATION_CPU, shape)
            total = used + free
            if total == 0:
                continue
            lines.append(f"[cpu (shape {shape}, {slabs} slabs)] {free} / {total} "
                         f"({free / total * 100:.2f}%) free; {moving} / {total} "
                         f"({moving / total * 100:.2f}%) moving; ")
        lines.append("---------------------------------")
        logger.info("\n".join(lines))
