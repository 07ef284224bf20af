"""Node-wide KV block manager on the native bookkeeping (``aegkv_bm_*``).

:class:`BlockManager` keeps the constructor, method names, arguments, errors
and controller-facing members of the reference's ``BlockManager``
(aegaeon/aegaeon/block_manager.py:165-874: ``cudart``, ``start_event_loop``,
``clear_zombie_requests``, ``latest_events``, ``zombie_request_ids``) and hands
out the same block ids in the same order.  The bookkeeping — GPU FIFO free
lists, the CPU slab pool, block tables and pending moves — lives in
``libaegkv.so``; this class keeps what is asynchronous or Python-side in the
reference: the per-engine swap callables, the move events' completion handles
and the reclaim's waiting.

Reclaim.  When an allocation runs short while moves out of that space are
pending, the native call suspends (it keeps its partial work, as the
reference's coroutine does across its ``await``) and names the space and the
last pending serial.  The ``async`` methods then do what ``_reclaim_blocks``
does (block_manager.py:360-472): await each pending move's handles, polling
them every ``SLEEP_WHEN_RECLAIM_PENDS`` seconds so the event loop keeps
running other coroutines, reclaim each move as it completes, then run the
slab pass for a CPU space, and resume the call.  A second coroutine that
needs the same space while a reclaim runs waits for that reclaim's lock, as
``move_gpu_locks`` / ``move_cpu_locks`` do.  The synchronous forms
(``allocate_blocks_by_count``, ``move_request_ids``) block on the handles
instead.

A move's handle (what the engine's remote callable returned for
``swap_blocks``) may be: None; an object with ``query()`` (a torch/HIP event;
the reference's ``cudaEventQuery``); an interprocess move handle of
:mod:`aegaeon_amd.swap_pool` (``rebuild_cuda_event``); an awaitable resolving
to handles (the reference's Ray object refs); a list of these; an object with
``synchronize()``; or a callable that returns once the copy is done.  A move
one of whose requests has finished counts as done (block_manager.py:373-376).
"""
from __future__ import annotations

import asyncio
import ctypes
import inspect
import logging
import math
import time
from dataclasses import dataclass
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

from . import _lib

logger = logging.getLogger(__name__)

BLOCK_LOCATION_CPU = -1  # block_manager.py:96
BLOCK_SIZE = 16          # aegaeon/aegaeon/config.py:13
SLEEP_IN_DAEMON_LOOP = 8            # block_manager.py:20
SLEEP_WHEN_RECLAIM_PENDS = 0.01     # block_manager.py:23
_NO_SPACE = -9
_IN_USE = -10
_RECLAIM = -12


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


def _is_ipc_handle(h) -> bool:
    return isinstance(h, tuple) and len(h) == 5 and isinstance(h[2], (bytes, bytearray))


def _wait_handle(h) -> None:
    """Block until the copy behind handle ``h`` is done."""
    if h is None:
        return
    if _is_ipc_handle(h):
        from . import swap_pool
        while not swap_pool.query_event(h):
            time.sleep(SLEEP_WHEN_RECLAIM_PENDS)
    elif isinstance(h, (list, tuple)):
        for x in h:
            _wait_handle(x)
    elif inspect.isawaitable(h):
        raise TypeError("an awaitable move handle needs the async API (allocate_blocks_batched, "
                        "move_requests)")
    elif hasattr(h, "synchronize"):
        h.synchronize()
    elif callable(h):
        h()
    else:
        raise TypeError(f"cannot wait on move handle {h!r}")


async def _resolve(h):
    """Await what is awaitable in a handle (the reference gathers its Ray
    futures first, MoveEvent._gather_event_handles, block_manager.py:136-142)."""
    while inspect.isawaitable(h):
        h = await h
    if isinstance(h, list):
        return [await _resolve(x) for x in h]
    if isinstance(h, tuple) and not _is_ipc_handle(h):
        return tuple([await _resolve(x) for x in h])
    return h


def _poll(h) -> Optional[bool]:
    """Whether the copy behind ``h`` is done, without blocking; None when the
    handle cannot be polled (it is then waited on)."""
    if h is None:
        return True
    if _is_ipc_handle(h):
        from . import swap_pool
        return swap_pool.query_event(h)
    if isinstance(h, (list, tuple)):
        states = [_poll(x) for x in h]
        if any(s is False for s in states):
            return False
        return None if any(s is None for s in states) else True
    if hasattr(h, "query"):
        return bool(h.query())
    return None


class BlockManager:
    """Drop-in for the reference's ``BlockManager`` (block_manager.py:165).

    ``wait_move(ev)`` replaces the waiting on a move's handles (it may return
    an awaitable); ``clear_zombies(ids)`` replaces the controller's
    ``remote_call_all_workers_async("clear_request_resource_batched", ids)``
    (block_manager.py:770-776); by default every registered engine's remote
    callable is called with that method."""

    def __init__(self, cpu_num_slabs: int, cpu_slab_size_bytes: int, dtype_size: int = 2,
                 wait_move: Optional[Callable[[MoveEvent], Any]] = None,
                 clear_zombies: Optional[Callable[[List[int]], Any]] = None):
        self.block_size = BLOCK_SIZE
        self.dtype_size = dtype_size
        self.cpu_num_slabs = cpu_num_slabs
        self.cpu_slab_size_bytes = cpu_slab_size_bytes
        self._lib = _lib.load()
        self._wait_move = wait_move
        self._clear_zombies = clear_zombies
        self._cudart = None
        self._h = None
        self._create()

    def _create(self) -> None:
        h = ctypes.c_void_p()
        _lib.check(self._lib.aegkv_bm_create(self.cpu_num_slabs, self.cpu_slab_size_bytes,
                                             ctypes.byref(h)), "BlockManager")
        self._h = h.value
        self._shape_ids: Dict[Tuple[int, ...], int] = {}
        self._shapes: List[Tuple[int, ...]] = []
        self.gpu_block_shape: Dict[int, Tuple[int, ...]] = {}
        self.gpu_num_max_blocks: Dict[int, int] = {}
        self.remote_callables: Dict[int, Callable] = {}
        self._moves: Dict[int, MoveEvent] = {}
        self._claimed: set = set()                 # serials a running reclaim awaits
        self._locks: Dict[tuple, asyncio.Event] = {}  # move_gpu_locks / move_cpu_locks
        self.latest_events: Dict[int, Any] = {}
        self.zombie_request_ids: List[int] = []

    def __del__(self):
        h, self._h = getattr(self, "_h", None), None
        if h:
            self._lib.aegkv_bm_destroy(h)

    @property
    def cudart(self):
        """The HIP runtime under ``CudaRTLibrary``'s method names (the
        reference creates one per manager, block_manager.py:182, and the
        controller uses it at llm.py:386-395)."""
        if self._cudart is None:
            from .hip_runtime import HipRTLibrary
            self._cudart = HipRTLibrary()
        return self._cudart

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

    def _check(self, rc: int, op: str, msg: str = "") -> None:
        if rc == 0:
            return
        if rc == _NO_SPACE:
            raise ResourceWarning(msg or f"{op}: not enough free blocks")
        if rc == _IN_USE:
            raise ValueError(msg or f"{op}: {_lib.strerror(rc)}")
        _lib.check(rc, op)

    # -- reclaim (block_manager.py:360-472) -----------------------------------------
    def _pending_moves(self, location: int, shape_id: int, serial: int) -> List[int]:
        shape = self._shapes[shape_id] if 0 <= shape_id < len(self._shapes) else None
        return sorted(s for s, ev in self._moves.items()
                      if s <= serial and ev.source_location == location
                      and (is_gpu(location) or ev.block_shape == shape))

    def _complete_move(self, location: int, shape_id: int, serial: int) -> None:
        _lib.check(self._lib.aegkv_bm_complete_move(self._h, location, shape_id, serial),
                   "complete_move")
        self._moves.pop(serial, None)

    def _finished(self, ev: MoveEvent) -> bool:
        return any(getattr(r, "is_finished", False) for r in ev.requests)

    async def _await_move(self, ev: MoveEvent) -> None:
        """Until the move's copy is done (the inner loop of _reclaim_blocks)."""
        if self._wait_move is not None:
            if not self._finished(ev):
                r = self._wait_move(ev)
                if inspect.isawaitable(r):
                    await r
            return
        while not self._finished(ev):
            ev.event_handle_refs = await _resolve(ev.event_handle_refs)
            state = _poll(ev.event_handle_refs)
            if state is None:
                _wait_handle(ev.event_handle_refs)
                return
            if state:
                return
            await asyncio.sleep(SLEEP_WHEN_RECLAIM_PENDS)

    async def _reclaim(self, location: int, shape_id: int, serial: int) -> None:
        """_reclaim_gpu/cpu_move_blocks: await and reclaim the pending moves out
        of the space up to ``serial`` that no other reclaim holds; with none
        left, wait for the reclaim that holds them."""
        key = (location,) if is_gpu(location) else (location, shape_id)
        mine = [s for s in self._pending_moves(location, shape_id, serial)
                if s not in self._claimed]
        if not mine:
            lock = self._locks.get(key)
            if lock is not None:
                await lock.wait()
            return
        lock = asyncio.Event()
        self._locks[key] = lock
        self._claimed.update(mine)
        try:
            for s in mine:
                ev = self._moves.get(s)
                if ev is not None:
                    await self._await_move(ev)
                self._complete_move(location, shape_id, s)
                self._claimed.discard(s)
            if not is_gpu(location):
                _lib.check(self._lib.aegkv_bm_reclaim_slabs(self._h), "reclaim_slabs")
            logger.debug("reclaimed %d move events of location %d", len(mine), location)
        finally:
            self._claimed.difference_update(mine)
            lock.set()

    def _reclaim_blocking(self, location: int, shape_id: int, serial: int) -> None:
        moves = self._pending_moves(location, shape_id, serial)
        for s in moves:
            ev = self._moves.get(s)
            if ev is not None and not self._finished(ev):
                if self._wait_move is not None:
                    r = self._wait_move(ev)
                    if inspect.isawaitable(r):
                        raise TypeError("wait_move returned an awaitable: use the async API")
                else:
                    _wait_handle(ev.event_handle_refs)
            self._complete_move(location, shape_id, s)
        if not is_gpu(location):
            _lib.check(self._lib.aegkv_bm_reclaim_slabs(self._h), "reclaim_slabs")

    def _pending(self) -> Tuple[int, int, int, int]:
        op, loc, sid, serial = (ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32(),
                                ctypes.c_int64())
        _lib.check(self._lib.aegkv_bm_pending(self._h, ctypes.byref(op), ctypes.byref(loc),
                                              ctypes.byref(sid), ctypes.byref(serial)),
                   "pending")
        return op.value, loc.value, sid.value, serial.value

    def _resume(self, op: int, out) -> int:
        return self._lib.aegkv_bm_resume(self._h, op, *[ctypes.byref(v) for v in out])

    def _cancel(self, op: int) -> None:
        if self._h:
            self._lib.aegkv_bm_cancel(self._h, op)

    def _drive_blocking(self, rc: int, out) -> int:
        while rc == _RECLAIM:
            op, loc, sid, serial = self._pending()
            try:
                self._reclaim_blocking(loc, sid, serial)
            except BaseException:
                self._cancel(op)
                raise
            rc = self._resume(op, out)
        return rc

    async def _drive(self, rc: int, out) -> int:
        while rc == _RECLAIM:
            op, loc, sid, serial = self._pending()
            try:
                await self._reclaim(loc, sid, serial)
            except BaseException:
                self._cancel(op)
                raise
            rc = self._resume(op, out)
        return rc

    # -- GPU spaces (:300-348, :600-602) ---------------------------------------
    def register_gpu_space(self, engine_id: int, num_max_blocks: int, block_shape,
                           remote_callable: Optional[Callable] = None) -> None:
        sid = self._shape_id(block_shape)
        rc = self._lib.aegkv_bm_register_gpu_space(self._h, engine_id, num_max_blocks, sid)
        self._check(rc, "register_gpu_space",
                    f"Error registering new GPU cache space for engine_id {engine_id}; "
                    "a request still resides in the cache, or a suspended call uses it.")
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

    _ALLOC_IN_USE = ("request is allocated elsewhere (migrate it before allocating more "
                     "blocks) or held by a suspended call")

    def _allocate_start(self, request_ids, num_blocks_needed, engine_id: int) -> int:
        ids, need = _i64(request_ids), _i64(num_blocks_needed)
        if ids.shape != need.shape:
            raise ValueError("one count per request")
        return self._lib.aegkv_bm_allocate(self._h, engine_id, _ptr(ids), _ptr(need), ids.size)

    @staticmethod
    def _out():
        return [ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int32(), ctypes.c_int32()]

    def allocate_blocks_by_count(self, request_ids: Sequence[int], num_blocks_needed: Sequence[int],
                                 engine_id: int) -> None:
        """allocate_blocks_batched with the totals already computed; a reclaim
        it needs blocks on the pending moves' handles."""
        rc = self._drive_blocking(self._allocate_start(request_ids, num_blocks_needed, engine_id),
                                  self._out())
        self._check(rc, "allocate_blocks_batched", self._ALLOC_IN_USE if rc == _IN_USE else "")

    async def allocate_blocks_by_count_async(self, request_ids: Sequence[int],
                                             num_blocks_needed: Sequence[int],
                                             engine_id: int) -> None:
        rc = await self._drive(self._allocate_start(request_ids, num_blocks_needed, engine_id),
                               self._out())
        self._check(rc, "allocate_blocks_batched", self._ALLOC_IN_USE if rc == _IN_USE else "")

    async def allocate_blocks_batched(self, batched_requests, engine_id: int) -> None:
        reqs = _requests_of(batched_requests)
        if len(reqs) == 0:
            return
        await self.allocate_blocks_by_count_async([r.request_id for r in reqs],
                                                  [self.get_num_blocks_needed(r) for r in reqs],
                                                  engine_id)

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
    def _move_start(self, request_ids: Sequence[int], target_location: int, out) -> int:
        ids = _i64(request_ids)
        return self._lib.aegkv_bm_move(self._h, _ptr(ids), ids.size, target_location,
                                       *[ctypes.byref(v) for v in out])

    def _move_result(self, rc: int, n_requests: int, out):
        if rc == -6:
            raise NotImplementedError("Migration is not implemented")
        if rc == -2:
            raise AssertionError("request not allocated")
        self._check(rc, "move_requests",
                    "a request of the move is held by a suspended call" if rc == _IN_USE else "")
        serial, nb, swap_in, engine = (v.value for v in out)
        if serial < 0:
            return None
        src = np.empty(nb, dtype=np.int64)
        dst = np.empty(nb, dtype=np.int64)
        moved = np.empty(n_requests, dtype=np.int64)
        n_moved = ctypes.c_int64()
        self._check(self._lib.aegkv_bm_move_ids(self._h, _ptr(src), _ptr(dst), src.size,
                                                _ptr(moved), moved.size, ctypes.byref(n_moved)),
                    "move_requests")
        src_ids = src.tolist()
        # pending until reclaimed; move_requests attaches the requests and handles
        self._moves[serial] = MoveEvent(serial, [], self.gpu_block_shape[engine],
                                        BLOCK_LOCATION_CPU if swap_in else engine,
                                        engine if swap_in else BLOCK_LOCATION_CPU, src_ids)
        return (serial, moved[:n_moved.value].tolist(), src_ids, dst.tolist(),
                bool(swap_in), engine)

    def move_request_ids(self, request_ids: Sequence[int], target_location: int):
        """The bookkeeping half of move_requests: returns ``None`` when nothing
        moves, else ``(serial, moved_request_ids, source_block_ids,
        target_block_ids, is_swap_in, engine_id)`` for the swap call.  A
        reclaim it needs blocks on the pending moves' handles."""
        out = self._out()
        rc = self._drive_blocking(self._move_start(request_ids, target_location, out), out)
        return self._move_result(rc, len(request_ids), out)

    async def move_request_ids_async(self, request_ids: Sequence[int], target_location: int):
        out = self._out()
        rc = await self._drive(self._move_start(request_ids, target_location, out), out)
        return self._move_result(rc, len(request_ids), out)

    async def move_requests(self, requests, target_location: int) -> bool:
        reqs = list(_requests_of(requests))
        res = await self.move_request_ids_async([r.request_id for r in reqs], target_location)
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

    # -- the controller's daemon (:351-358, :770-776) ------------------------------
    async def start_event_loop(self):
        """Runs forever: every SLEEP_IN_DAEMON_LOOP seconds log the block usage
        and clear the zombie requests (block_manager.py:351-358)."""
        while True:
            await asyncio.sleep(SLEEP_IN_DAEMON_LOOP)
            self.log_block_usage()
            self.clear_zombie_requests()

    def clear_zombie_requests(self) -> None:
        """Tell the workers to drop the freed requests' move events
        (``clear_request_resource_batched``), then forget them."""
        ids = list(self.zombie_request_ids)
        if self._clear_zombies is not None:
            self._clear_zombies(ids)
        else:
            for remote in self.remote_callables.values():
                if remote is not None:
                    remote("clear_request_resource_batched", ids)
        self.zombie_request_ids.clear()

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
