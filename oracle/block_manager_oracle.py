"""Pure-Python restatement of the reference's block-manager bookkeeping
(aegaeon/aegaeon/block_manager.py) — test infrastructure that the native
block manager's results are compared with, never on the product path.

Restated synchronously: where the reference awaits the completion of pending
moves (_reclaim_blocks, block_manager.py:360-408), this class calls
``wait(location, block_shape, serial)``, which returns once every move out of
that location up to ``serial`` has finished copying.  Ray calls, CUDA events,
``latest_events`` and zombie lists are left out: they do not change which ids
are handed out.  Everything else keeps the reference's data structures and
order: FIFO GPU free lists (list slicing), per-shape CPU deques, a free-slab
stack, the float ``ceil``/``floor`` slab ranges, and the defect of
``register_gpu_space`` that clears every engine's pending GPU moves
(block_manager.py:321-322).

Parity pins (no reference tests exist for this file): literal known-answer
sequences worked out by hand from the cited lines, and conservation
invariants (every block of a space is free, in exactly one table, or moving).
"""
from __future__ import annotations

import math
from collections import defaultdict, deque
from dataclasses import dataclass, field
from typing import Callable, Deque, Dict, List, Optional, Sequence, Tuple

BLOCK_LOCATION_CPU = -1  # block_manager.py:96
BLOCK_SIZE = 16          # aegaeon/aegaeon/config.py:13


def is_gpu(location: int) -> bool:
    return location >= 0  # block_manager.py:99-100


@dataclass
class BlockTable:  # block_manager.py:103-111
    location: int
    block_shape: Tuple[int, ...]
    blocks: List[int]


@dataclass(eq=False)
class MoveEvent:  # block_manager.py:114-131, without the CUDA event handles
    serial: int
    request_ids: List[int]
    block_shape: Tuple[int, ...]
    source_location: int
    target_location: int
    source_blocks: List[int]


@dataclass
class MoveResult:
    """What move_requests hands to the swap call (block_manager.py:839-846)."""
    moved: bool
    request_ids: List[int] = field(default_factory=list)
    source_block_ids: List[int] = field(default_factory=list)
    target_block_ids: List[int] = field(default_factory=list)
    is_swap_in: bool = False
    engine_id: Optional[int] = None
    serial: int = -1


class BlockManagerOracle:
    """block_manager.py:165-874 without the asynchronous plumbing."""

    def __init__(self, cpu_num_slabs: int, cpu_slab_size_bytes: int, dtype_size: int = 2,
                 wait: Optional[Callable[[int, Tuple[int, ...], int], bool]] = None):
        # block_manager.py:180-237
        self.block_size = BLOCK_SIZE
        self.dtype_size = dtype_size
        self.serial = 0
        self.cpu_num_slabs = cpu_num_slabs
        self.cpu_slab_size_bytes = cpu_slab_size_bytes
        self.cpu_free_blocks: Dict[Tuple[int, ...], Deque[int]] = defaultdict(deque)
        self.cpu_free_slabs: List[int] = list(range(cpu_num_slabs))
        self.cpu_slab_usage: List[int] = [0] * cpu_num_slabs
        self.cpu_block_shape: List[Optional[Tuple[int, ...]]] = [None] * cpu_num_slabs
        self.gpu_block_shape: Dict[int, Tuple[int, ...]] = {}
        self.gpu_num_max_blocks: Dict[int, int] = {}
        self.gpu_free_blocks: Dict[int, List[int]] = {}
        self.move_events_cpu: Dict[Tuple[int, ...], Deque[MoveEvent]] = defaultdict(deque)
        self.move_cpu_num_blocks: Dict[Tuple[int, ...], int] = defaultdict(int)
        self.move_events_gpu: Dict[int, Deque[MoveEvent]] = defaultdict(deque)
        self.move_gpu_num_blocks: Dict[int, int] = {}
        self.block_tables: Dict[int, BlockTable] = {}
        self.wait = wait if wait is not None else (lambda loc, shape, serial: True)

    # -- helpers ------------------------------------------------------------
    def _get_block_size_bytes(self, block_shape) -> int:  # :239-240
        return math.prod(block_shape) * self.dtype_size

    def _get_slab_range(self, slab: int, block_size_bytes: int) -> Tuple[int, int]:  # :242-245
        start = math.ceil(slab * self.cpu_slab_size_bytes / block_size_bytes)
        end = math.floor((slab + 1) * self.cpu_slab_size_bytes / block_size_bytes)
        return start, end

    def _slab_of(self, block: int, block_size_bytes: int) -> int:  # :269-270
        return block * block_size_bytes // self.cpu_slab_size_bytes

    def _reclaim_gpu_move_blocks_once(self, ev: MoveEvent) -> int:  # :247-258
        self.move_gpu_num_blocks[ev.source_location] -= len(ev.source_blocks)
        self.gpu_free_blocks[ev.source_location].extend(ev.source_blocks)
        return len(ev.source_blocks)

    def _reclaim_cpu_move_blocks_once(self, ev: MoveEvent) -> int:  # :260-272
        bb = self._get_block_size_bytes(ev.block_shape)
        self.move_cpu_num_blocks[ev.block_shape] -= len(ev.source_blocks)
        self.cpu_free_blocks[ev.block_shape].extend(ev.source_blocks)
        for block in ev.source_blocks:
            self.cpu_slab_usage[self._slab_of(block, bb)] -= 1
        return len(ev.source_blocks)

    # -- register (:300-348) -------------------------------------------------
    def register_gpu_space(self, engine_id: int, num_max_blocks: int, block_shape) -> None:
        block_shape = tuple(block_shape)
        if self.gpu_free_blocks.get(engine_id) is not None:
            for req_id, bt in self.block_tables.items():
                if bt.location == engine_id:
                    raise ValueError(f"request {req_id} still resides in engine {engine_id}")
        if engine_id in self.move_events_gpu:
            self.move_events_gpu.clear()  # every engine's (:321-322)
        self.move_gpu_num_blocks[engine_id] = 0
        old = self.gpu_block_shape.get(engine_id)
        if old is not None:
            q = self.move_events_cpu[old]
            for _ in range(len(q)):
                ev = q[0]
                if ev.target_location == engine_id:
                    q.popleft()
                    self._reclaim_cpu_move_blocks_once(ev)
                else:
                    q.rotate(-1)
        self.gpu_block_shape[engine_id] = block_shape
        self.gpu_num_max_blocks[engine_id] = num_max_blocks
        self.gpu_free_blocks[engine_id] = list(range(num_max_blocks))

    # -- reclaim (:360-496) --------------------------------------------------
    def _reclaim_blocks(self, move_events: Deque[MoveEvent], target_serial: int,
                        location: int, block_shape, once) -> None:
        if not self.wait(location, block_shape, target_serial):
            raise ResourceWarning("pending moves did not finish")
        while move_events and move_events[0].serial <= target_serial:
            once(move_events.popleft())

    def _reclaim_gpu_move_blocks(self, location: int, block_shape) -> None:  # :410-436
        q = self.move_events_gpu[location]
        if q:
            self._reclaim_blocks(q, q[-1].serial, location, block_shape,
                                 self._reclaim_gpu_move_blocks_once)

    def _reclaim_cpu_move_blocks(self, block_shape) -> None:  # :438-472
        q = self.move_events_cpu[block_shape]
        if q:
            self._reclaim_blocks(q, q[-1].serial, BLOCK_LOCATION_CPU, block_shape,
                                 self._reclaim_cpu_move_blocks_once)
            self._reclaim_cpu_slabs()

    def _reclaim_cpu_slabs(self) -> bool:  # :474-496
        reclaimed = 0
        for slab, usage in enumerate(self.cpu_slab_usage):
            shape = self.cpu_block_shape[slab]
            if usage == 0 and shape is not None:
                reclaimed += 1
                bb = self._get_block_size_bytes(shape)
                fl = self.cpu_free_blocks[shape]
                start, end = self._get_slab_range(slab, bb)
                for _ in range(len(fl)):
                    block = fl[0]
                    if start <= block < end:
                        fl.popleft()
                    else:
                        fl.rotate(-1)
                self.cpu_free_slabs.append(slab)
                self.cpu_block_shape[slab] = None
        return reclaimed > 0

    # -- allocation (:498-598) -----------------------------------------------
    def _get_free_blocks(self, num_blocks: int, location: int, block_shape) -> List[int]:
        bb = self._get_block_size_bytes(block_shape)
        if is_gpu(location):
            assert location in self.gpu_free_blocks, f"unknown gpu location {location}"
            fl = self.gpu_free_blocks[location]
            if len(fl) < num_blocks:
                self._reclaim_gpu_move_blocks(location, block_shape)
                if len(fl) < num_blocks:
                    raise ResourceWarning("not enough free blocks on GPU")
            blocks = fl[:num_blocks]
            fl[:] = fl[num_blocks:]
            return blocks
        fl = self.cpu_free_blocks[block_shape]

        def ensure_slab_blocks(needed: int) -> bool:
            if needed <= 0:
                return True
            for slab in self.cpu_free_slabs:
                assert self.cpu_block_shape[slab] is None
                start, end = self._get_slab_range(slab, bb)
                needed -= end - start
                if needed <= 0:
                    return True
            return False

        if not ensure_slab_blocks(num_blocks - len(fl)):
            self._reclaim_cpu_move_blocks(block_shape)
            if not ensure_slab_blocks(num_blocks - len(fl)):
                raise ResourceWarning("not enough free blocks on CPU")
        while len(fl) < num_blocks:
            slab = self.cpu_free_slabs.pop()
            start, end = self._get_slab_range(slab, bb)
            self.cpu_block_shape[slab] = block_shape
            fl.extend(range(start, end))
        blocks = []
        for _ in range(num_blocks):
            block = fl.popleft()
            self.cpu_slab_usage[self._slab_of(block, bb)] += 1
            blocks.append(block)
        return blocks

    def _get_free_blocks_batched(self, nums: Sequence[int], location: int, block_shape):
        free = self._get_free_blocks(sum(nums), location, block_shape)  # :584-598
        out, cur = [], 0
        for n in nums:
            out.append(free[cur:cur + n])
            cur += n
        return out

    def get_num_blocks_needed(self, n_tokens: int) -> int:  # :604-609
        return (n_tokens + self.block_size - 1) // self.block_size

    def allocate_blocks_batched(self, requests: Sequence[Tuple[int, int]], engine_id: int):
        """``requests``: (request_id, total blocks needed) pairs (:651-694)."""
        if len(requests) == 0:
            return
        shape = self.gpu_block_shape[engine_id]
        nums = []
        for rid, needed in requests:
            bt = self.block_tables.get(rid)
            assert bt is None or bt.location == engine_id, f"request {rid} is elsewhere"
            nums.append(needed if bt is None else needed - len(bt.blocks))
        lists = self._get_free_blocks_batched(nums, engine_id, shape)
        for (rid, _), blocks in zip(requests, lists):
            if rid not in self.block_tables:
                self.block_tables[rid] = BlockTable(engine_id, shape, blocks)
            else:
                self.block_tables[rid].blocks.extend(blocks)

    def free_blocks(self, request_id: int) -> None:  # :696-711
        bt = self.block_tables.pop(request_id)
        if is_gpu(bt.location):
            self.gpu_free_blocks[bt.location].extend(bt.blocks)
        else:
            bb = self._get_block_size_bytes(bt.block_shape)
            self.cpu_free_blocks[bt.block_shape].extend(bt.blocks)
            for block in bt.blocks:
                self.cpu_slab_usage[self._slab_of(block, bb)] -= 1

    # -- moves (:778-874) ----------------------------------------------------
    def move_requests(self, request_ids: Sequence[int], target_location: int) -> MoveResult:
        swapped: List[int] = []
        cur_loc: Optional[int] = None
        shape = None
        engine = None
        src_ids: List[int] = []
        dst_ids: List[int] = []
        for rid in request_ids:
            bt = self.block_tables.get(rid)
            assert bt is not None, f"request {rid} not allocated"
            if bt.location == target_location:
                continue
            if is_gpu(bt.location) and is_gpu(target_location):
                raise NotImplementedError("Migration is not implemented")
            if cur_loc is not None:
                assert bt.location == cur_loc
            if shape is not None:
                assert bt.block_shape == shape
            cur_loc = bt.location
            shape = bt.block_shape
            swapped.append(rid)
            engine = target_location if is_gpu(target_location) else cur_loc
            new = self._get_free_blocks(len(bt.blocks), target_location, shape)
            src_ids += bt.blocks
            dst_ids += new
            bt.blocks = new
            bt.location = target_location
        if not swapped:
            return MoveResult(False)
        ev = MoveEvent(self.serial, swapped, shape, cur_loc, target_location, src_ids)
        self.serial += 1
        if is_gpu(cur_loc):
            self.move_gpu_num_blocks[cur_loc] += len(src_ids)
            self.move_events_gpu[cur_loc].append(ev)
        else:
            self.move_cpu_num_blocks[shape] += len(src_ids)
            self.move_events_cpu[shape].append(ev)
        return MoveResult(True, swapped, src_ids, dst_ids, is_gpu(target_location), engine,
                          ev.serial)

    # -- views for tests -----------------------------------------------------
    def stats(self, location: int, block_shape=None) -> Tuple[int, int, int, int]:
        """(free, moving, slabs, used) as log_block_usage counts them (:730-768)."""
        if is_gpu(location):
            return (len(self.gpu_free_blocks[location]), self.move_gpu_num_blocks[location], 0, 0)
        shape = tuple(block_shape)
        slabs = [i for i, s in enumerate(self.cpu_block_shape) if s == shape]
        return (len(self.cpu_free_blocks.get(shape, ())), self.move_cpu_num_blocks.get(shape, 0),
                len(slabs), sum(self.cpu_slab_usage[i] for i in slabs))

    def free_list(self, location: int, block_shape=None) -> List[int]:
        if is_gpu(location):
            return list(self.gpu_free_blocks[location])
        return list(self.cpu_free_blocks.get(tuple(block_shape), ()))
