"""Block manager: the oracle pinned by hand-worked cases and conservation
invariants, then the native bookkeeping (aegkv_bm_*) against the oracle on
random operation sequences — same tables, same free-list order, same swap id
lists.  Host code only: these run without a GPU."""
import asyncio
import copy
import math
from dataclasses import dataclass

import numpy as np
import pytest

from aegaeon_amd.block_manager import BLOCK_LOCATION_CPU as CPU, BlockManager
from oracle.block_manager_oracle import BlockManagerOracle

SHAPE_A = (16, 2, 4, 8)   # 1024 elements -> 2048 bytes per block
SHAPE_B = (16, 3, 4, 8)   # 3072 bytes per block: straddles 8 KiB slab edges
SHAPE_C = (15,)           # 30 bytes per block


# ---------------------------------------------------------------------------
# oracle pins
# ---------------------------------------------------------------------------
def test_oracle_gpu_fifo_literal():
    """Head-take / tail-append order (block_manager.py:515-526,703)."""
    o = BlockManagerOracle(0, 1)
    o.register_gpu_space(0, 8, SHAPE_A)
    o.allocate_blocks_batched([(1, 3), (2, 2)], 0)
    assert o.block_tables[1].blocks == [0, 1, 2]
    assert o.block_tables[2].blocks == [3, 4]
    o.free_blocks(1)
    assert o.free_list(0) == [5, 6, 7, 0, 1, 2]
    o.allocate_blocks_batched([(3, 4)], 0)
    assert o.block_tables[3].blocks == [5, 6, 7, 0]
    o.allocate_blocks_batched([(2, 4)], 0)          # grows at the tail of its table
    assert o.block_tables[2].blocks == [3, 4, 1, 2]
    with pytest.raises(ResourceWarning):
        o.allocate_blocks_batched([(4, 1)], 0)


def test_oracle_cpu_slab_literal():
    """30-byte blocks in 100-byte slabs: slab s holds ids ceil(100 s / 30) ..
    floor(100 (s + 1) / 30) - 1, i.e. {0,1,2}, {4,5}, {7,8,9}, {10,11,12};
    free slabs are popped from the back of [0, 1, 2, 3] (block_manager.py:566-570)."""
    o = BlockManagerOracle(4, 100)
    o.register_gpu_space(0, 10, SHAPE_C)
    o.allocate_blocks_batched([(1, 4)], 0)
    r = o.move_requests([1], CPU)
    assert r.source_block_ids == [0, 1, 2, 3]
    assert r.target_block_ids == [10, 11, 12, 7]     # slab 3, then slab 2
    assert not r.is_swap_in and r.engine_id == 0 and r.serial == 0
    assert o.cpu_free_slabs == [0, 1]
    assert o.cpu_slab_usage == [0, 0, 1, 3]
    assert o.free_list(CPU, SHAPE_C) == [8, 9]
    assert o.stats(0) == (6, 4, 0, 0)                # 4 GPU blocks moving out
    # swap back in: takes GPU blocks 4..7; the CPU blocks are now moving
    r = o.move_requests([1], 0)
    assert r.target_block_ids == [4, 5, 6, 7] and r.is_swap_in and r.serial == 1
    assert o.stats(CPU, SHAPE_C) == (2, 4, 2, 4)
    # 6 GPU blocks needed, 2 free: the swap-out's sources are reclaimed first
    o.allocate_blocks_batched([(2, 2), (3, 4)], 0)
    assert o.block_tables[2].blocks == [8, 9] and o.block_tables[3].blocks == [0, 1, 2, 3]
    assert o.stats(0) == (0, 0, 0, 0)
    # 10 CPU blocks: [8, 9] from the deque, slabs 1 and 0 for request 3, then
    # request 1 runs short, the swap-in is reclaimed, slab 3 returns and is reused
    r = o.move_requests([2, 3, 1], CPU)
    assert r.request_ids == [2, 3, 1] and r.serial == 2
    assert r.source_block_ids == [8, 9, 0, 1, 2, 3, 4, 5, 6, 7]
    assert r.target_block_ids == [8, 9, 4, 5, 0, 1, 2, 7, 10, 11]
    assert o.cpu_slab_usage == [3, 2, 3, 2] and o.cpu_free_slabs == []
    assert o.free_list(CPU, SHAPE_C) == [12]
    # GPU: reclaim of serial 2 gives [8, 9] to request 4, [0] to request 5
    o.allocate_blocks_batched([(4, 2), (5, 1)], 0)
    assert o.block_tables[4].blocks == [8, 9] and o.block_tables[5].blocks == [0]
    with pytest.raises(ResourceWarning):
        o.move_requests([5, 4], CPU)                  # 3 CPU blocks, 1 left
    # the reference leaves request 5 moved when request 4 fails (its defect)
    assert o.block_tables[5].location == CPU and o.block_tables[5].blocks == [12]
    assert o.block_tables[4].location == 0


def test_oracle_cpu_reclaim_returns_slabs_in_order():
    o = BlockManagerOracle(4, 100)
    o.register_gpu_space(0, 10, SHAPE_C)
    o.allocate_blocks_batched([(1, 4)], 0)
    o.move_requests([1], CPU)                         # CPU ids [10, 11, 12, 7]
    o.move_requests([1], 0)                           # CPU blocks moving
    o.allocate_blocks_batched([(2, 2)], 0)            # unrelated GPU allocation
    o.allocate_blocks_batched([(3, 1)], 0)
    r = o.move_requests([2], CPU)                     # 2 needed, deque [8, 9] has them
    assert r.target_block_ids == [8, 9]
    r = o.move_requests([3], CPU)                     # needs 1: ensure -> slabs [0, 1] ok
    assert r.target_block_ids == [4]                  # slab 1 popped: {4, 5}
    assert o.cpu_free_slabs == [0]
    o._reclaim_cpu_move_blocks(SHAPE_C)               # the swap-in of request 1 finished
    # slab 3 (ids 10-12) is empty now; slab 2 still holds 8, 9 -> only slab 3 returns
    assert o.cpu_free_slabs == [0, 3]
    assert o.free_list(CPU, SHAPE_C) == [5, 7]


def _check_invariants(o: BlockManagerOracle):
    """Every block of a space is free, in exactly one table, or moving."""
    for e, n in o.gpu_num_max_blocks.items():
        free = o.free_list(e)
        used = [b for t in o.block_tables.values() if t.location == e for b in t.blocks]
        moving = [b for ev in o.move_events_gpu.get(e, ()) for b in ev.source_blocks]
        everything = free + used + moving
        assert sorted(everything) == list(range(n)), e
        assert o.move_gpu_num_blocks[e] == len(moving)
    usage = [0] * o.cpu_num_slabs
    for shape in set(list(o.cpu_free_blocks) + [t.block_shape for t in o.block_tables.values()]):
        bb = math.prod(shape) * o.dtype_size
        used = [b for t in o.block_tables.values() if t.location == CPU and t.block_shape == shape
                for b in t.blocks]
        moving = [b for ev in o.move_events_cpu.get(shape, ()) for b in ev.source_blocks]
        free = o.free_list(CPU, shape)
        allb = used + moving + free
        assert len(set(allb)) == len(allb)
        for b in allb:
            slab = b * bb // o.cpu_slab_size_bytes
            # the block lies wholly inside one slab that holds this shape
            assert (b + 1) * bb <= (slab + 1) * o.cpu_slab_size_bytes
            assert o.cpu_block_shape[slab] == shape
        for b in used + moving:
            usage[b * bb // o.cpu_slab_size_bytes] += 1
        assert o.move_cpu_num_blocks.get(shape, 0) == len(moving)
    assert usage == o.cpu_slab_usage
    for s in o.cpu_free_slabs:
        assert o.cpu_block_shape[s] is None


# ---------------------------------------------------------------------------
# random driver
# ---------------------------------------------------------------------------
class _Sim:
    """Drives the oracle and the native manager with the same operations."""

    def __init__(self, seed, n_slabs=24, slab_bytes=8192, engines=((0, 40, SHAPE_A),
                                                                   (1, 30, SHAPE_B))):
        self.rng = np.random.default_rng(seed)
        self.o = BlockManagerOracle(n_slabs, slab_bytes)
        self.n = BlockManager(n_slabs, slab_bytes)
        self.engines = {}
        for e, nmax, shape in engines:
            self.register(e, nmax, shape)
        self.next_id = 0
        self.results = []

    def register(self, e, nmax, shape):
        self.o.register_gpu_space(e, nmax, shape)
        self.n.register_gpu_space(e, nmax, shape)
        self.engines[e] = shape

    def compare(self):
        o, n = self.o, self.n
        for rid in range(self.next_id):
            t = o.block_tables.get(rid)
            if t is None:
                with pytest.raises(AssertionError):
                    n.get_block_table(rid)
                continue
            nt = n.get_block_table(rid)
            assert (nt.location, nt.block_shape, nt.blocks) == (t.location, t.block_shape,
                                                                t.blocks), rid
        for e in self.engines:
            assert n.free_list(e) == o.free_list(e), e
            assert n.stats(e) == o.stats(e), e
        for shape in set(self.engines.values()):
            assert n.free_list(CPU, shape) == o.free_list(CPU, shape), shape
            assert n.stats(CPU, shape) == o.stats(CPU, shape), shape
        _check_invariants(o)

    def step(self):
        o, n, rng = self.o, self.n, self.rng
        op = rng.choice(["alloc", "grow", "free", "out", "in", "rereg"],
                        p=[0.3, 0.2, 0.15, 0.15, 0.15, 0.05])
        gpu_reqs = [r for r, t in o.block_tables.items() if t.location >= 0]
        cpu_reqs = [r for r, t in o.block_tables.items() if t.location == CPU]
        if op == "alloc" or (op == "grow" and not gpu_reqs):
            e = int(rng.choice(list(self.engines)))
            k = int(rng.integers(1, 5))
            reqs = [(self.next_id + i, int(rng.integers(0, 6))) for i in range(k)]
            self.next_id += k
            self._alloc(reqs, e)
        elif op == "grow":
            e = o.block_tables[int(rng.choice(gpu_reqs))].location
            mine = [r for r in gpu_reqs if o.block_tables[r].location == e]
            pick = rng.choice(mine, size=min(len(mine), int(rng.integers(1, 4))), replace=False)
            self._alloc([(int(r), len(o.block_tables[int(r)].blocks) + int(rng.integers(0, 3)))
                         for r in pick], e)
        elif op == "free":
            if o.block_tables:
                rid = int(rng.choice(list(o.block_tables)))
                o.free_blocks(rid)
                n.free_blocks(rid)
        elif op == "out" and gpu_reqs:
            e = o.block_tables[int(rng.choice(gpu_reqs))].location
            mine = [r for r in gpu_reqs if o.block_tables[r].location == e]
            pick = [int(r) for r in rng.choice(mine, size=min(len(mine), int(rng.integers(1, 4))),
                                               replace=False)]
            self._move(pick, CPU)
        elif op == "in" and cpu_reqs:
            r0 = int(rng.choice(cpu_reqs))
            shape = o.block_tables[r0].block_shape
            targets = [e for e, s in self.engines.items() if s == shape]
            if targets:
                mine = [r for r in cpu_reqs if o.block_tables[r].block_shape == shape]
                pick = [int(r) for r in rng.choice(mine, size=min(len(mine),
                                                                 int(rng.integers(1, 4))),
                                                   replace=False)]
                self._move(pick, int(rng.choice(targets)))
        elif op == "rereg":
            e = int(rng.choice(list(self.engines)))
            empty = all(t.location != e for t in o.block_tables.values())
            # the reference drops every engine's pending GPU moves here; keep
            # to the cases where that and the native form agree
            others_idle = all(len(q) == 0 for k, q in o.move_events_gpu.items() if k != e)
            if empty and others_idle:
                shape = [SHAPE_A, SHAPE_B, SHAPE_C][int(rng.integers(0, 3))]
                self.register(e, int(rng.integers(10, 50)), shape)
        self.compare()

    def _alloc(self, reqs, e):
        try:
            self.o.allocate_blocks_batched(reqs, e)
            ok = True
        except ResourceWarning:
            ok = False
        if ok:
            self.n.allocate_blocks_by_count([r for r, _ in reqs], [c for _, c in reqs], e)
        else:
            with pytest.raises(ResourceWarning):
                self.n.allocate_blocks_by_count([r for r, _ in reqs], [c for _, c in reqs], e)

    def _move(self, pick, target):
        trial = copy.deepcopy(self.o)
        try:
            trial.move_requests(pick, target)
        except ResourceWarning:
            return  # the reference leaves a failed batch half-moved: not compared
        r = self.o.move_requests(pick, target)
        got = self.n.move_request_ids(pick, target)
        if not r.moved:
            assert got is None
            return
        serial, moved, src, dst, swap_in, engine = got
        assert (serial, moved, src, dst, swap_in, engine) == (
            r.serial, r.request_ids, r.source_block_ids, r.target_block_ids, r.is_swap_in,
            r.engine_id)
        self.results.append(len(src))


@pytest.mark.parametrize("seed", range(12))
def test_native_matches_oracle_random(seed):
    sim = _Sim(seed)
    for _ in range(250):
        sim.step()
    assert sum(sim.results) > 0  # moves happened


def test_native_matches_oracle_tight_cpu_pool():
    """Few slabs: CPU allocations keep reclaiming slabs and running short."""
    sim = _Sim(99, n_slabs=6, slab_bytes=8192)
    for _ in range(400):
        sim.step()


def test_native_matches_oracle_straddling_blocks():
    """30-byte blocks in 100-byte slabs: blocks straddle every slab edge."""
    sim = _Sim(7, n_slabs=8, slab_bytes=100, engines=((0, 16, SHAPE_C), (1, 12, SHAPE_C)))
    for _ in range(300):
        sim.step()


# ---------------------------------------------------------------------------
# native behaviour beyond the reference
# ---------------------------------------------------------------------------
def test_move_rollback_restores_free_list_order():
    """Slabs {0,1,2} and {4,5}: requests 1 and 2 get [4, 5] and [0, 1], request
    3 (3 blocks) finds one left and fails; the native manager puts the taken
    blocks back at the head of the deque in order and restores the tables."""
    n = BlockManager(2, 100)
    n.register_gpu_space(0, 12, SHAPE_C)
    n.allocate_blocks_by_count([1, 2, 3], [2, 2, 3], 0)
    tables = {r: n.get_block_table(r).blocks for r in (1, 2, 3)}
    assert tables == {1: [0, 1], 2: [2, 3], 3: [4, 5, 6]}
    with pytest.raises(ResourceWarning):
        n.move_request_ids([1, 2, 3], CPU)
    for r in (1, 2, 3):
        t = n.get_block_table(r)
        assert t.location == 0 and t.blocks == tables[r]
    assert n.free_list(CPU, SHAPE_C) == [4, 5, 0, 1, 2]
    assert n.stats(CPU, SHAPE_C) == (5, 0, 2, 0)      # both slabs open, none used
    assert n.free_list(0) == [7, 8, 9, 10, 11]
    got = n.move_request_ids([1, 2], CPU)
    assert got[1] == [1, 2] and got[2] == [0, 1, 2, 3] and got[3] == [4, 5, 0, 1]


def test_wait_failure_raises_and_reclaims_nothing():
    waited = []

    def wait_move(ev):
        waited.append(ev.serial)
        raise TimeoutError("copy still running")

    n = BlockManager(8, 8192, wait_move=wait_move)
    n.register_gpu_space(0, 4, SHAPE_A)
    n.allocate_blocks_by_count([1], [4], 0)
    asyncio.run(n.move_requests([_Req(1)], CPU))
    with pytest.raises(TimeoutError):
        n.allocate_blocks_by_count([2], [1], 0)       # needs the swap-out's blocks
    assert waited == [0]
    assert n.free_list(0) == [] and n.stats(0)[1] == 4
    n2 = BlockManager(8, 8192)                         # no handles: copies count as done
    n2.register_gpu_space(0, 4, SHAPE_A)
    n2.allocate_blocks_by_count([1], [4], 0)
    asyncio.run(n2.move_requests([_Req(1)], CPU))
    n2.allocate_blocks_by_count([2], [1], 0)
    assert n2.get_block_table(2).blocks == [0]


def test_reregister_keeps_other_engines_moves():
    """The reference clears every engine's pending GPU moves when an engine it
    has seen moves on re-registers (block_manager.py:321-322), stranding their
    source blocks; the native manager drops only that engine's."""
    n = BlockManager(16, 8192)
    o = BlockManagerOracle(16, 8192)
    for m in (n, o):
        m.register_gpu_space(0, 4, SHAPE_A)
        m.register_gpu_space(1, 4, SHAPE_A)
    n.allocate_blocks_by_count([9], [4], 1)
    o.allocate_blocks_batched([(9, 4)], 1)
    n.move_request_ids([9], CPU)                      # engine 1 has seen a move
    o.move_requests([9], CPU)
    n.allocate_blocks_by_count([10], [1], 1)          # reclaims it
    o.allocate_blocks_batched([(10, 1)], 1)
    for m in (n, o):
        m.free_blocks(10)
    n.allocate_blocks_by_count([1], [4], 0)
    o.allocate_blocks_batched([(1, 4)], 0)
    n.move_request_ids([1], CPU)                      # pending on engine 0
    o.move_requests([1], CPU)
    for m in (n, o):
        m.register_gpu_space(1, 4, SHAPE_A)
    n.allocate_blocks_by_count([2], [4], 0)           # reclaims engine 0's swap-out
    assert n.get_block_table(2).blocks == [0, 1, 2, 3]
    with pytest.raises(ResourceWarning):               # the reference lost those blocks
        o.allocate_blocks_batched([(2, 4)], 0)


def test_errors_mirror_the_reference():
    n = BlockManager(4, 8192)
    n.register_gpu_space(0, 8, SHAPE_A)
    n.register_gpu_space(1, 8, SHAPE_A)
    n.allocate_blocks_by_count([1], [2], 0)
    with pytest.raises(AssertionError):
        n.free_blocks(99)
    with pytest.raises(AssertionError):
        n.get_block_table(99)
    with pytest.raises(NotImplementedError):
        n.move_request_ids([1], 1)                    # GPU -> GPU migration
    with pytest.raises(ValueError):
        n.allocate_blocks_by_count([1], [3], 1)       # lives on engine 0
    with pytest.raises(ValueError):
        n.register_gpu_space(0, 8, SHAPE_A)           # request 1 still there
    assert n.move_request_ids([1], 0) is None         # already there: nothing moves


def test_flat_tables_feed_prepare_inputs_layout():
    n = BlockManager(0, 1)
    n.register_gpu_space(0, 64, SHAPE_A)
    n.allocate_blocks_by_count([5, 6, 7], [3, 0, 2], 0)
    n.free_blocks(5)
    n.allocate_blocks_by_count([8], [4], 0)
    offsets, ids = n.flat_block_tables([7, 6, 8])
    assert offsets.tolist() == [0, 2, 2, 6]
    assert ids.dtype == np.int32
    assert ids.tolist() == [3, 4, 5, 6, 7, 8]


# ---------------------------------------------------------------------------
# reference-shaped async API
# ---------------------------------------------------------------------------
@dataclass
class _Req:
    request_id: int
    n_in: int = 20
    n_out: int = 0
    is_finished: bool = False

    def get_input_len(self):
        return self.n_in

    def get_output_len(self):
        return self.n_out


@dataclass
class _Batch:
    requests: list

    def __len__(self):
        return len(self.requests)


def test_async_api_and_swap_callable():
    calls, waited = [], []

    def remote(method, req_ids, src, dst, handles, is_swap_in):
        calls.append((method, list(req_ids), list(src), list(dst), list(handles), is_swap_in))
        return [lambda: waited.append(tuple(req_ids))]

    n = BlockManager(4, 8192)
    n.register_gpu_space(0, 6, SHAPE_A, remote)
    reqs = [_Req(1, 20), _Req(2, 33)]                  # 2 and 3 blocks
    asyncio.run(n.allocate_blocks_batched(_Batch(reqs), 0))
    assert n.get_block_table(1).blocks == [0, 1] and n.get_block_table(2).blocks == [2, 3, 4]
    assert n.get_num_append_blocks_needed(_Req(1, 20, 13)) == 1
    assert asyncio.run(n.move_requests(_Batch(reqs), CPU))
    assert calls[0][0] == "swap_blocks" and calls[0][1] == [1, 2]
    assert calls[0][2] == [0, 1, 2, 3, 4] and calls[0][4] == [None, None]
    assert calls[0][5] is False
    assert not n.is_all_requests_on_gpu(_Batch(reqs))
    assert not asyncio.run(n.move_requests(_Batch(reqs), CPU))  # nothing moves
    asyncio.run(n.allocate_blocks_batched(_Batch([_Req(3, 40)]), 0))  # 3 blocks: [5] + reclaim
    assert waited == [(1, 2)]
    assert n.get_block_table(3).blocks == [5, 0, 1]
    # swap-in waits on nothing yet; its source handles are the swap-out's
    assert asyncio.run(n.move_requests([reqs[0]], 0))
    assert calls[1][1] == [1] and calls[1][5] is True and calls[1][4][0] is not None
    n.free_blocks_batched(reqs)
    assert n.zombie_request_ids == [1, 2]
    n.log_block_usage()
    n.reset()
    with pytest.raises(AssertionError):
        n.get_block_table(3)


# ---------------------------------------------------------------------------
# awaitable reclaim (block_manager.py:360-472) and the controller's members
# ---------------------------------------------------------------------------
class _Copy:
    """A move's handle whose copy finishes when the test says so (the
    reference polls cudaEventQuery on it, block_manager.py:387-398)."""

    def __init__(self):
        self.done = False
        self.polls = 0

    def query(self):
        self.polls += 1
        return self.done


def _copies_remote(copies):
    def remote(method, *args):
        assert method == "swap_blocks"
        c = _Copy()
        copies.append(c)
        return c
    return remote


def test_reclaim_awaits_while_other_coroutines_run():
    """An allocation that needs a pending swap-out's blocks awaits its copy
    without blocking the event loop: another engine allocates and finishes
    meanwhile; the ids are the oracle's."""
    copies, log = [], []
    n = BlockManager(4, 8192)
    o = BlockManagerOracle(4, 8192)
    n.register_gpu_space(0, 4, SHAPE_A, _copies_remote(copies))
    n.register_gpu_space(1, 6, SHAPE_A, _copies_remote(copies))
    for m in (o,):
        m.register_gpu_space(0, 4, SHAPE_A)
        m.register_gpu_space(1, 6, SHAPE_A)
    r1 = _Req(1, 64)                                      # 4 blocks
    asyncio.run(n.allocate_blocks_batched(_Batch([r1]), 0))
    o.allocate_blocks_batched([(1, 4)], 0)
    assert asyncio.run(n.move_requests(_Batch([r1]), CPU))
    o.move_requests([1], CPU)
    assert len(copies) == 1 and not copies[0].done

    async def needs_reclaim():
        await n.allocate_blocks_batched(_Batch([_Req(2, 32)]), 0)   # 2 blocks: reclaim
        log.append("engine 0 allocated")

    async def other_engine():
        for i in range(4):
            await n.allocate_blocks_batched(_Batch([_Req(10 + i, 16)]), 1)
            log.append(f"engine 1 step {i}")
            await asyncio.sleep(0.02)
        copies[0].done = True                             # the swap-out's copy ends

    async def main():
        await asyncio.gather(needs_reclaim(), other_engine())

    asyncio.run(main())
    assert log == [f"engine 1 step {i}" for i in range(4)] + ["engine 0 allocated"]
    assert copies[0].polls >= 3                           # polled, not blocked on
    o.allocate_blocks_batched([(2, 2)], 0)
    o.allocate_blocks_batched([(10 + i, 1) for i in range(4)], 1)
    for rid in (2, 10, 11, 12, 13):
        assert n.get_block_table(rid).blocks == o.block_tables[rid].blocks, rid
    assert n.free_list(0) == o.free_list(0) and n.stats(0) == o.stats(0)


def test_mid_move_cpu_reclaim_awaited_matches_oracle():
    """The oracle's hand-worked sequence (slabs of 30-byte blocks), with every
    move's copy finishing only after the reclaim has started waiting: the
    swap-out of [2, 3, 1] runs short at request 1, awaits the swap-in's copy,
    reclaims its CPU blocks and slab 3, and continues with the same ids."""
    copies = []
    n = BlockManager(4, 100)
    o = BlockManagerOracle(4, 100)
    n.register_gpu_space(0, 10, SHAPE_C, _copies_remote(copies))
    o.register_gpu_space(0, 10, SHAPE_C)
    req = {i: _Req(i, 16 * k) for i, k in ((1, 4), (2, 2), (3, 4))}

    async def finish_later(k, delay=0.03):
        await asyncio.sleep(delay)
        copies[k].done = True

    async def run(coro, k):
        await asyncio.gather(coro, finish_later(k))

    asyncio.run(n.allocate_blocks_batched(_Batch([req[1]]), 0))
    o.allocate_blocks_batched([(1, 4)], 0)
    asyncio.run(n.move_requests([req[1]], CPU))       # copy 0: swap-out
    o.move_requests([1], CPU)
    asyncio.run(n.move_requests([req[1]], 0))         # copy 1: swap-in
    o.move_requests([1], 0)
    # 6 GPU blocks, 2 free: awaits copy 0 (the swap-out) before reclaiming
    asyncio.run(run(n.allocate_blocks_batched(_Batch([req[2], req[3]]), 0), 0))
    o.allocate_blocks_batched([(2, 2), (3, 4)], 0)
    for rid in (2, 3):
        assert n.get_block_table(rid).blocks == o.block_tables[rid].blocks
    # the swap-out of [2, 3, 1] needs a CPU reclaim after 2 and 3 took blocks
    result = {}

    async def move():
        result["moved"] = await n.move_requests([req[2], req[3], req[1]], CPU)

    asyncio.run(run(move(), 1))
    r = o.move_requests([2, 3, 1], CPU)
    assert result["moved"]
    for rid in (1, 2, 3):
        t = n.get_block_table(rid)
        assert (t.location, t.blocks) == (o.block_tables[rid].location,
                                          o.block_tables[rid].blocks), rid
    assert n.get_block_table(2).blocks + n.get_block_table(3).blocks + \
        n.get_block_table(1).blocks == r.target_block_ids == [8, 9, 4, 5, 0, 1, 2, 7, 10, 11]
    assert n.free_list(CPU, SHAPE_C) == o.free_list(CPU, SHAPE_C) == [12]
    assert n.stats(CPU, SHAPE_C) == o.stats(CPU, SHAPE_C)


def test_second_reclaimer_waits_for_the_first():
    """Two coroutines run short on the same engine: the first awaits the
    pending move, the second waits for the first's reclaim (its lock) and then
    takes the next blocks, in the order the oracle gives sequentially."""
    copies = []
    n = BlockManager(8, 8192)
    o = BlockManagerOracle(8, 8192)
    n.register_gpu_space(0, 6, SHAPE_A, _copies_remote(copies))
    o.register_gpu_space(0, 6, SHAPE_A)
    asyncio.run(n.allocate_blocks_batched(_Batch([_Req(1, 64), _Req(2, 32)]), 0))
    o.allocate_blocks_batched([(1, 4), (2, 2)], 0)
    asyncio.run(n.move_requests([_Req(1, 64)], CPU))
    o.move_requests([1], CPU)

    async def finish():
        await asyncio.sleep(0.03)
        copies[0].done = True

    async def main():
        await asyncio.gather(n.allocate_blocks_batched(_Batch([_Req(3, 32)]), 0),
                             n.allocate_blocks_batched(_Batch([_Req(4, 16)]), 0), finish())

    asyncio.run(main())
    o.allocate_blocks_batched([(3, 2)], 0)
    o.allocate_blocks_batched([(4, 1)], 0)
    for rid in (3, 4):
        assert n.get_block_table(rid).blocks == o.block_tables[rid].blocks, rid
    assert n.free_list(0) == o.free_list(0)


def test_suspended_move_holds_its_requests_and_cancel_undoes_it():
    """While a move waits for a reclaim, its requests are busy (another
    allocation or move of them is refused); cancelling the waiting coroutine
    undoes the move, tables and free lists as before it."""
    copies = []
    n = BlockManager(1, 6 * 2048)                    # one slab: 6 CPU blocks of SHAPE_A
    n.register_gpu_space(0, 16, SHAPE_A, _copies_remote(copies))
    reqs = [_Req(1, 64), _Req(2, 32), _Req(3, 64)]   # 4 + 2 + 4 blocks
    asyncio.run(n.allocate_blocks_batched(_Batch(reqs), 0))
    before = {r.request_id: n.get_block_table(r.request_id).blocks for r in reqs}
    asyncio.run(n.move_requests([reqs[0]], CPU))     # CPU 0..3, copy 0 pending
    asyncio.run(n.move_requests([reqs[0]], 0))       # swap-in: CPU blocks moving (copy 1)
    free_cpu = n.free_list(CPU, SHAPE_A)
    free_gpu = n.free_list(0)
    tables = {r.request_id: n.get_block_table(r.request_id).blocks for r in reqs}

    async def main():
        # 2 then 4 CPU blocks: request 2 fits, request 3 waits for copy 1
        task = asyncio.ensure_future(n.move_requests([reqs[1], reqs[2]], CPU))
        await asyncio.sleep(0.03)
        assert not task.done()
        assert n.get_block_table(2).location == CPU  # moved before the wait
        with pytest.raises(ValueError):
            await n.allocate_blocks_batched(_Batch([reqs[1]]), 0)
        with pytest.raises(ValueError):
            await n.move_requests([reqs[2]], CPU)
        task.cancel()
        with pytest.raises(asyncio.CancelledError):
            await task

    asyncio.run(main())
    for r in reqs:
        t = n.get_block_table(r.request_id)
        assert t.location == 0 and t.blocks == tables[r.request_id]
    assert n.free_list(CPU, SHAPE_A) == free_cpu and n.free_list(0) == free_gpu
    assert before[2] == tables[2] and before[3] == tables[3]
    copies[1].done = True                             # now the same move goes through
    assert asyncio.run(n.move_requests([reqs[1], reqs[2]], CPU))
    assert n.get_block_table(3).location == CPU


def test_free_during_suspended_move_drops_the_request():
    """A request freed while its move waits leaves the move: its target
    blocks went back with the free, its source blocks are freed at the
    source, and the swap lists carry only the others."""
    copies, calls = [], []
    n = BlockManager(1, 6 * 2048)
    remote = _copies_remote(copies)

    def recording(method, *args):
        calls.append(args)
        return remote(method, *args)

    n.register_gpu_space(0, 16, SHAPE_A, recording)
    reqs = [_Req(1, 64), _Req(2, 32), _Req(3, 64)]
    asyncio.run(n.allocate_blocks_batched(_Batch(reqs), 0))
    asyncio.run(n.move_requests([reqs[0]], CPU))
    asyncio.run(n.move_requests([reqs[0]], 0))
    gpu_of_2 = n.get_block_table(2).blocks

    async def main():
        task = asyncio.ensure_future(n.move_requests([reqs[1], reqs[2]], CPU))
        await asyncio.sleep(0.03)
        n.free_blocks(2)                             # moved already, then freed
        copies[1].done = True
        assert await task

    asyncio.run(main())
    ids, src, dst = calls[-1][0], calls[-1][1], calls[-1][2]
    assert ids == [3] and len(src) == len(dst) == 4
    assert n.get_block_table(3).location == CPU
    assert set(gpu_of_2) <= set(n.free_list(0))      # request 2's GPU blocks are free
    free_cpu = n.free_list(CPU, SHAPE_A)
    assert len(set(free_cpu)) == len(free_cpu)


def test_sync_api_blocks_on_query_handles():
    """allocate_blocks_by_count (the blocking form) waits on a handle that has
    only query()/synchronize() and gives the same ids."""
    class _Ev:
        def __init__(self):
            self.synced = False

        def query(self):
            return self.synced

        def synchronize(self):
            self.synced = True

    evs = []

    def remote(method, *args):
        evs.append(_Ev())
        return evs[-1]

    n = BlockManager(4, 8192)
    n.register_gpu_space(0, 4, SHAPE_A, remote)
    n.allocate_blocks_by_count([1], [4], 0)
    asyncio.run(n.move_requests([_Req(1, 64)], CPU))
    n.allocate_blocks_by_count([2], [3], 0)
    assert evs[0].synced and n.get_block_table(2).blocks == [0, 1, 2]


def test_controller_members(monkeypatch, tmp_path):
    """What the reference's controller touches after
    ``block_manager = BlockManager(cpu_num_slabs, cpu_slab_size_bytes)``
    (llm.py:383-395, 486-499): ``cudart`` with CudaRTLibrary's methods, the
    swap space, and ``start_event_loop`` in the controller's asyncio.gather,
    which logs usage and clears zombies every SLEEP_IN_DAEMON_LOOP seconds."""
    import aegaeon_amd.block_manager as bmod
    from aegaeon_amd import swap_pool
    n = BlockManager(2, 1 << 16)
    for name in ("cudaSetDevice", "cudaDeviceSynchronize", "cudaDeviceReset",
                 "cudaGetErrorString", "cudaMalloc", "cudaHostRegister", "cudaFree",
                 "cudaMemset", "cudaMemcpy", "cudaIpcGetMemHandle", "cudaIpcOpenMemHandle",
                 "cudaIpcCloseMemHandle", "cudaIpcGetEventHandle", "cudaIpcOpenEventHandle",
                 "cudaStreamWaitEvent", "cudaEventSynchronize", "cudaEventQuery",
                 "cudaEventDestroy", "CUDART_CHECK"):
        assert callable(getattr(n.cudart, name)), name
    assert n.cudart.cudaGetErrorString(0) == "no error"
    cache = swap_pool.init_cpu_cache(2, 1 << 16, str(tmp_path / "cpu_cache"))
    assert cache.numel() * 2 == 2 << 16
    cleared = []
    worker_side = []

    def remote(method, *args):
        worker_side.append((method, args))

    n.register_gpu_space(0, 8, SHAPE_A, remote)
    monkeypatch.setattr(bmod, "SLEEP_IN_DAEMON_LOOP", 0.01)

    async def engine():
        await n.allocate_blocks_batched(_Batch([_Req(1, 20), _Req(2, 20)]), 0)
        n.free_blocks_batched([_Req(1), _Req(2)])
        await asyncio.sleep(0.05)
        raise KeyboardInterrupt  # ends the controller's gather

    async def controller():
        await asyncio.gather(n.start_event_loop(), engine())

    with pytest.raises(KeyboardInterrupt):
        asyncio.run(controller())
    assert ("clear_request_resource_batched", ([1, 2],)) in worker_side
    assert n.zombie_request_ids == []
    n2 = BlockManager(2, 1 << 16, clear_zombies=cleared.append)
    n2.register_gpu_space(0, 8, SHAPE_A)
    n2.allocate_blocks_by_count([5], [1], 0)
    n2.free_blocks(5)
    n2.clear_zombie_requests()
    assert cleared == [[5]] and n2.zombie_request_ids == []
