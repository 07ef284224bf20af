"""The move protocol end to end on the GPU: the native block manager and the
oracle manager driven through the same random sequence of allocations,
decode steps, swap-outs, swap-ins and frees (reclaim included), with every
move's id lists fed through the workers' swap streams and events
(aegaeon/aegaeon/block_manager.py:474-874, worker.py:473-500,716-815).

Two engines with different block shapes (16 KiB and 24 KiB blocks) share one
CPU swap space cut into slabs, as the reference's engines share the node's
swap file: a slab holds blocks of one shape while it is used and returns to
the free-slab stack when emptied, so the other shape reuses it
(block_manager.py:474-582).  The 24 KiB blocks straddle the 64 KiB slab edges.

Each stream is held behind a spin before its work, so an order that only
held by luck would show: the append on the compute stream is still pending
when the swap-out is enqueued (the swap-out must wait on the append's event
and carry the appended token to the host); a swap-in is still pending when
the next decode step is enqueued (the step must wait on its event); a
swap-out is still pending when the manager reclaims its source blocks (the
reclaim must wait on the move's event before the blocks are written again).
With ``async_api`` the allocations and moves go through the coroutine API,
whose reclaim polls the move events from the event loop.

A host model (the oracle's append, swap and attention on numpy copies of the
pools) follows the same operations; the GPU pools, the pinned swap space and
every decode attention must match it: bytes bit-exact, attention within 2e-3
relative L2 (and one output ulp elementwise) of the float64 textbook."""
import asyncio
import copy
import math
from dataclasses import dataclass

import numpy as np
import pytest
import torch

from aegaeon_amd import attention as A
from aegaeon_amd.block_manager import BLOCK_LOCATION_CPU as CPU, BlockManager
from aegaeon_amd.worker_swap import KVSwapWorker
from oracle import kv_oracle as ko
from oracle.block_manager_oracle import BlockManagerOracle
from tests.kvtest_utils import bf16_ulp, random_bits, to_bits, to_device_bits

pytestmark = pytest.mark.gpu

H, D, HQ = 2, 64, 4
SHAPES = {0: (2, 2, 16, H, D),          # engine 0: 2 layers, 16 KiB blocks (bf16)
          1: (3, 2, 16, H, D)}          # engine 1: 3 layers, 24 KiB blocks
N_GPU = {0: 40, 1: 28}
SLAB = 64 << 10                         # 4 blocks of 16 KiB, or 2 of 24 KiB
N_SLABS = 8
HOLD = 1_000_000                        # spin cycles (~1 ms) put in front of a stream's work


def _bb(shape):
    return int(np.prod(shape)) * 2


@dataclass
class _Req:
    request_id: int
    is_finished: bool = False


def _check_attention(got_bits, ref):
    got = ko.bits_to_float(got_bits, "bf16")
    err = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= 2e-3, err
    assert not (np.abs(got - ref) > bf16_ulp(ref) + 1e-5).any()


class _Engine:
    def __init__(self, run, e):
        self.e, self.shape = e, SHAPES[e]
        self.layers = self.shape[0]
        dev = run.dev
        self.compute = torch.cuda.Stream(device=dev)
        self.cache = torch.zeros((N_GPU[e], *self.shape), dtype=torch.bfloat16, device=dev)
        n_cpu = N_SLABS * SLAB // _bb(self.shape)
        per = int(np.prod(self.shape))
        # the shared swap space seen with this engine's block shape (worker.py:134-142)
        self.swap = run.swap[:n_cpu * per].view(n_cpu, *self.shape)
        self.model_gpu = np.zeros((N_GPU[e], *self.shape), dtype=np.uint16)
        self.model_cpu = run.model_swap[:n_cpu * per].reshape(n_cpu, *self.shape)
        self.worker = KVSwapWorker(self.cache, self.swap, self.compute)
        self.last_append = None
        remote = self.worker.remote_callable(lambda: self.last_append)

        def recording_remote(method, *args):
            if method == "swap_blocks":
                rids, src, dst, handles, is_swap_in = args
                run.calls.append((self.e, list(rids), list(src), list(dst), is_swap_in))
            return remote(method, *args)

        self.remote = recording_remote


class _Run:
    def __init__(self, device, seed, async_api=False):
        self.dev = device
        self.async_api = async_api
        self.rng = np.random.default_rng(seed)
        self.swap = torch.zeros(N_SLABS * SLAB // 2, dtype=torch.bfloat16, pin_memory=True)
        self.model_swap = np.zeros(N_SLABS * SLAB // 2, dtype=np.uint16)
        self.calls = []
        self.engines = {e: _Engine(self, e) for e in SHAPES}
        self.bm = BlockManager(N_SLABS, SLAB)
        self.orc = BlockManagerOracle(N_SLABS, SLAB)
        for e, eng in self.engines.items():
            self.bm.register_gpu_space(e, N_GPU[e], eng.shape, eng.remote)
            self.orc.register_gpu_space(e, N_GPU[e], eng.shape)
        self.lens = {}                    # request id -> tokens held
        self.engine_of = {}               # request id -> engine whose shape it has
        self.next_id = 0
        self.counts = {"out": 0, "in": 0, "decode": 0, "attn_waited": 0, "reclaims": 0,
                       "slab_reuse": 0}
        self.slab_shapes = {}

    # -- helpers -----------------------------------------------------------------
    def where(self, rid):
        return self.orc.block_tables[rid].location

    def table(self, rid):
        t = self.bm.get_block_table(rid)
        assert (t.location, t.blocks) == (self.orc.block_tables[rid].location,
                                          self.orc.block_tables[rid].blocks), rid
        return t.blocks

    def note_slabs(self):
        """Count slabs that changed block shape (cross-shape reuse)."""
        for s, shape in enumerate(self.orc.cpu_block_shape):
            if shape is None:
                continue
            if self.slab_shapes.get(s, shape) != shape:
                self.counts["slab_reuse"] += 1
            self.slab_shapes[s] = shape

    def allocate(self, pairs, e):
        """Both managers, same outcome; False when the pool runs short."""
        n_moving_before = self.orc.stats(e)[1]
        ids, need = [r for r, _ in pairs], [c for _, c in pairs]
        try:
            self.orc.allocate_blocks_batched(pairs, e)
        except ResourceWarning:
            with pytest.raises(ResourceWarning):
                self._bm_allocate(ids, need, e)
            return False
        self._bm_allocate(ids, need, e)
        if self.orc.stats(e)[1] < n_moving_before:
            self.counts["reclaims"] += 1
        return True

    def _bm_allocate(self, ids, need, e):
        if self.async_api:
            asyncio.run(self.bm.allocate_blocks_by_count_async(ids, need, e))
        else:
            self.bm.allocate_blocks_by_count(ids, need, e)

    def append(self, eng, rids, positions_per_req):
        """K/V rows for the given positions of each request, on the held
        compute stream; the model follows."""
        slots = []
        for rid, pos in zip(rids, positions_per_req):
            t = self.table(rid)
            slots.extend(t[p // 16] * 16 + p % 16 for p in pos)
        T = len(slots)
        key = random_bits(self.rng, (eng.layers, T, H, D), "bf16")
        val = random_bits(self.rng, (eng.layers, T, H, D), "bf16")
        slots = np.asarray(slots, dtype=np.int64)
        ko.append_layers(key, val, eng.model_gpu, slots)
        with torch.cuda.stream(eng.compute):
            kd, vd = to_device_bits(key, "bf16", self.dev), to_device_bits(val, "bf16", self.dev)
            sd = torch.from_numpy(slots).to(self.dev)
            torch.cuda._sleep(HOLD)
            A.append_kv(kd, vd, eng.cache, sd)
            ev = torch.cuda.Event()
            ev.record(eng.compute)
            # the host buffers of this step live until the stream is past them
            for t in (kd, vd, sd):
                t.record_stream(eng.compute)
        eng.last_append = ev

    # -- operations ----------------------------------------------------------------
    def new_requests(self):
        e = int(self.rng.integers(0, len(SHAPES)))
        k = int(self.rng.integers(1, 3))
        lens = [int(x) for x in self.rng.integers(1, 48, k)]
        rids = list(range(self.next_id, self.next_id + k))
        self.next_id += k
        if not self.allocate([(r, -(-n // 16)) for r, n in zip(rids, lens)], e):
            return
        for r, n in zip(rids, lens):
            self.lens[r] = n
            self.engine_of[r] = e
        self.append(self.engines[e], rids, [range(n) for n in lens])

    def decode(self):
        e = int(self.rng.integers(0, len(SHAPES)))
        eng = self.engines[e]
        gpu = [r for r in self.lens if self.where(r) == e]
        if not gpu:
            return
        mask = eng.worker.wait_for_moves(gpu, eng.compute)
        if not all(eng.worker.ready_mask(gpu)):
            self.counts["attn_waited"] += 1
        run = [r for r, ok in zip(gpu, mask) if ok]
        if not self.allocate([(r, -(-(self.lens[r] + 1) // 16)) for r in run], e):
            return
        self.append(eng, run, [[self.lens[r]] for r in run])
        for r in run:
            self.lens[r] += 1
        tables = [self.table(r) for r in run]
        lens = np.asarray([self.lens[r] for r in run], dtype=np.int64)
        padded = ko.pad_block_tables(tables)
        q = random_bits(self.rng, (len(run), HQ, D), "bf16")
        scale = 1 / math.sqrt(D)
        view = eng.cache.permute(1, 2, 0, 3, 4, 5)
        with torch.cuda.stream(eng.compute):
            qd = to_device_bits(q, "bf16", self.dev)
            bt = torch.from_numpy(padded).to(self.dev)
            sl = torch.from_numpy(lens.astype(np.int32)).to(self.dev)
            outs = [A.paged_decode_attention(qd, view[l, 0], view[l, 1], bt, sl, scale,
                                             int(lens.max())) for l in range(eng.layers)]
        eng.compute.synchronize()
        mv = eng.model_gpu.transpose(1, 2, 0, 3, 4, 5)
        for l in range(eng.layers):
            ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"),
                                            ko.bits_to_float(mv[l, 0], "bf16"),
                                            ko.bits_to_float(mv[l, 1], "bf16"), padded, lens,
                                            scale)
            _check_attention(to_bits(outs[l]), ref)
        self.counts["decode"] += 1

    def move(self, to_cpu):
        if to_cpu:
            e = int(self.rng.integers(0, len(SHAPES)))
            here = [r for r in self.lens if self.where(r) == e]
            target = CPU
        else:
            here = [r for r in self.lens if self.where(r) == CPU]
            if here:
                e = self.engine_of[int(self.rng.choice(here))]
                here = [r for r in here if self.engine_of[r] == e]
            target = e if here else None
        if not here:
            return
        eng = self.engines[e]
        pick = [int(r) for r in self.rng.choice(here, size=min(len(here),
                                                               int(self.rng.integers(1, 4))),
                                                replace=False)]
        trial = copy.deepcopy(self.orc)
        try:
            trial.move_requests(pick, target)
        except ResourceWarning:
            return                     # the reference leaves such a batch half moved
        res = self.orc.move_requests(pick, target)
        stream = eng.worker.swap_out_stream if to_cpu else eng.worker.swap_in_stream
        with torch.cuda.stream(stream):
            torch.cuda._sleep(HOLD)    # the move is still in flight afterwards
        n_calls = len(self.calls)
        moved = asyncio.run(self.bm.move_requests([_Req(r) for r in pick], target))
        assert moved == res.moved
        if not res.moved:
            assert len(self.calls) == n_calls
            return
        # the swap the worker ran carries the oracle's lists
        assert self.calls[-1] == (e, res.request_ids, res.source_block_ids,
                                  res.target_block_ids, res.is_swap_in)
        for r in res.request_ids:
            self.table(r)                                 # same location and blocks
        ko.swap_blocks(res.source_block_ids, res.target_block_ids, res.is_swap_in,
                       eng.model_gpu, eng.model_cpu)
        self.counts["out" if to_cpu else "in"] += 1
        self.note_slabs()

    def free(self):
        if not self.lens:
            return
        rid = int(self.rng.choice(list(self.lens)))
        eng = self.engines[self.engine_of[rid]]
        # the scheduler frees a request only once its moves have finished
        for e in eng.worker.move_event_table.get(rid, []):
            e.synchronize()
        eng.compute.synchronize()
        self.orc.free_blocks(rid)
        self.bm.free_blocks(rid)
        eng.worker.clear_request_resource(rid)
        del self.lens[rid]

    def check_pools(self):
        torch.cuda.synchronize()
        for eng in self.engines.values():
            assert np.array_equal(to_bits(eng.cache), eng.model_gpu), eng.e
        assert np.array_equal(self.swap.view(torch.int16).numpy().view(np.uint16),
                              self.model_swap)


@pytest.mark.parametrize("seed,async_api", [(0, False), (1, False), (2, True), (3, True)])
def test_block_manager_moves_through_worker_streams(device, seed, async_api):
    run = _Run(device, seed, async_api)
    ops = ["new", "decode", "out", "in", "free"]
    p = [0.25, 0.33, 0.18, 0.16, 0.08]
    for i in range(120):
        op = ops[int(run.rng.choice(len(ops), p=p))]
        print(f"seed {seed} step {i}: {op}", flush=True)
        if op == "new":
            run.new_requests()
        elif op == "decode":
            run.decode()
        elif op == "out":
            run.move(True)
        elif op == "in":
            run.move(False)
        else:
            run.free()
        if i % 15 == 14:
            run.check_pools()
    run.check_pools()
    c = run.counts
    print(seed, c, flush=True)
    assert c["out"] >= 3 and c["in"] >= 3 and c["decode"] >= 10, c
