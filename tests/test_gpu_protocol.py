"""The move protocol end to end on the GPU: the native block manager and the
oracle manager driven through the same random sequence of allocations,
decode steps, swap-outs, swap-ins and frees (reclaim included), with every
move's id lists fed through the worker's swap streams and events
(aegaeon/aegaeon/block_manager.py:651-874, worker.py:473-500,716-815).

Each stream is held behind a spin before its work, so an order that only
held by luck would show: the append on the compute stream is still pending
when the swap-out is enqueued (the swap-out must wait on the append's event
and carry the appended token to the host); a swap-in is still pending when
the next decode step is enqueued (the step must wait on its event); a
swap-out is still pending when the manager reclaims its source blocks (the
reclaim must wait on the move's event before the blocks are written again).

A host model (the oracle's append, swap and attention on numpy copies of both
pools) follows the same operations; the GPU pool, the pinned swap space and
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

L, H, D, HQ = 2, 2, 64, 4
SHAPE = (L, 2, 16, H, D)                 # 16 KiB blocks (bf16)
BB = int(np.prod(SHAPE)) * 2
N_GPU = 40
N_SLABS, SLAB = 6, 4 * BB                # 24 CPU blocks, 4 per slab
HOLD = 1_000_000                         # spin cycles (~1 ms) put in front of a stream's work


@dataclass
class _Req:
    request_id: int
    is_finished: bool = False


def _check_attention(got_bits, ref):
    got = ko.bits_to_float(got_bits, "bf16")
    err = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= 2e-3, err
    assert not (np.abs(got - ref) > bf16_ulp(ref) + 1e-5).any()


class _Run:
    def __init__(self, device, seed):
        self.dev = device
        self.rng = np.random.default_rng(seed)
        self.compute = torch.cuda.Stream(device=device)
        self.cache = torch.zeros((N_GPU, *SHAPE), dtype=torch.bfloat16, device=device)
        self.swap = torch.zeros((N_SLABS * SLAB // BB, *SHAPE), dtype=torch.bfloat16,
                                pin_memory=True)
        self.model_gpu = np.zeros((N_GPU, *SHAPE), dtype=np.uint16)
        self.model_cpu = np.zeros(self.swap.shape, dtype=np.uint16)
        self.worker = KVSwapWorker(self.cache, self.swap, self.compute)
        self.last_append = None
        self.bm = BlockManager(N_SLABS, SLAB)
        remote = self.worker.remote_callable(lambda: self.last_append)
        self.calls = []

        def recording_remote(method, rids, src, dst, handles, is_swap_in):
            self.calls.append((list(rids), list(src), list(dst), is_swap_in))
            return remote(method, rids, src, dst, handles, is_swap_in)

        self.bm.register_gpu_space(0, N_GPU, SHAPE, recording_remote)
        self.orc = BlockManagerOracle(N_SLABS, SLAB)
        self.orc.register_gpu_space(0, N_GPU, SHAPE)
        self.lens = {}                    # request id -> tokens held
        self.next_id = 0
        self.counts = {"out": 0, "in": 0, "decode": 0, "attn_waited": 0, "reclaims": 0}

    # -- helpers -----------------------------------------------------------------
    def where(self, rid):
        return self.orc.block_tables[rid].location

    def table(self, rid):
        t = self.bm.get_block_table(rid)
        assert (t.location, t.blocks) == (self.orc.block_tables[rid].location,
                                          self.orc.block_tables[rid].blocks), rid
        return t.blocks

    def allocate(self, pairs):
        """Both managers, same outcome; False when the pool runs short."""
        n_moving_before = self.orc.stats(0)[1]
        try:
            self.orc.allocate_blocks_batched(pairs, 0)
        except ResourceWarning:
            with pytest.raises(ResourceWarning):
                self.bm.allocate_blocks_by_count([r for r, _ in pairs], [c for _, c in pairs], 0)
            return False
        self.bm.allocate_blocks_by_count([r for r, _ in pairs], [c for _, c in pairs], 0)
        if self.orc.stats(0)[1] < n_moving_before:
            self.counts["reclaims"] += 1
        return True

    def append(self, rids, positions_per_req):
        """K/V rows for the given positions of each request, on the held
        compute stream; the model follows."""
        slots = []
        for rid, pos in zip(rids, positions_per_req):
            t = self.table(rid)
            slots.extend(t[p // 16] * 16 + p % 16 for p in pos)
        T = len(slots)
        key = random_bits(self.rng, (L, T, H, D), "bf16")
        val = random_bits(self.rng, (L, T, H, D), "bf16")
        slots = np.asarray(slots, dtype=np.int64)
        ko.append_layers(key, val, self.model_gpu, slots)
        with torch.cuda.stream(self.compute):
            kd, vd = to_device_bits(key, "bf16", self.dev), to_device_bits(val, "bf16", self.dev)
            sd = torch.from_numpy(slots).to(self.dev)
            torch.cuda._sleep(HOLD)
            A.append_kv(kd, vd, self.cache, sd)
            ev = torch.cuda.Event()
            ev.record(self.compute)
            # the host buffers of this step live until the stream is past them
            for t in (kd, vd, sd):
                t.record_stream(self.compute)
        self.last_append = ev

    # -- operations ----------------------------------------------------------------
    def new_requests(self):
        k = int(self.rng.integers(1, 3))
        lens = [int(x) for x in self.rng.integers(1, 48, k)]
        rids = list(range(self.next_id, self.next_id + k))
        self.next_id += k
        if not self.allocate([(r, -(-n // 16)) for r, n in zip(rids, lens)]):
            return
        for r, n in zip(rids, lens):
            self.lens[r] = n
        self.append(rids, [range(n) for n in lens])

    def decode(self):
        gpu = [r for r in self.lens if self.where(r) >= 0]
        if not gpu:
            return
        mask = self.worker.wait_for_moves(gpu, self.compute)
        if not all(self.worker.ready_mask(gpu)):
            self.counts["attn_waited"] += 1
        run = [r for r, ok in zip(gpu, mask) if ok]
        if not self.allocate([(r, -(-(self.lens[r] + 1) // 16)) for r in run]):
            return
        self.append(run, [[self.lens[r]] for r in run])
        for r in run:
            self.lens[r] += 1
        tables = [self.table(r) for r in run]
        lens = np.asarray([self.lens[r] for r in run], dtype=np.int64)
        padded = ko.pad_block_tables(tables)
        q = random_bits(self.rng, (len(run), HQ, D), "bf16")
        scale = 1 / math.sqrt(D)
        view = self.cache.permute(1, 2, 0, 3, 4, 5)
        with torch.cuda.stream(self.compute):
            qd = to_device_bits(q, "bf16", self.dev)
            bt = torch.from_numpy(padded).to(self.dev)
            sl = torch.from_numpy(lens.astype(np.int32)).to(self.dev)
            outs = [A.paged_decode_attention(qd, view[l, 0], view[l, 1], bt, sl, scale,
                                             int(lens.max())) for l in range(L)]
        self.compute.synchronize()
        mv = self.model_gpu.transpose(1, 2, 0, 3, 4, 5)
        for l in range(L):
            ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"),
                                            ko.bits_to_float(mv[l, 0], "bf16"),
                                            ko.bits_to_float(mv[l, 1], "bf16"), padded, lens,
                                            scale)
            _check_attention(to_bits(outs[l]), ref)
        self.counts["decode"] += 1

    def move(self, target):
        here = [r for r in self.lens if (self.where(r) >= 0) == (target == CPU)]
        if not here:
            return
        pick = [int(r) for r in self.rng.choice(here, size=min(len(here),
                                                               int(self.rng.integers(1, 4))),
                                                replace=False)]
        trial = copy.deepcopy(self.orc)
        try:
            trial.move_requests(pick, target)
        except ResourceWarning:
            return                     # the reference leaves such a batch half moved
        res = self.orc.move_requests(pick, target)
        stream = self.worker.swap_in_stream if target >= 0 else self.worker.swap_out_stream
        with torch.cuda.stream(stream):
            torch.cuda._sleep(HOLD)    # the move is still in flight afterwards
        n_calls = len(self.calls)
        moved = asyncio.run(self.bm.move_requests([_Req(r) for r in pick], target))
        assert moved == res.moved
        if not res.moved:
            assert len(self.calls) == n_calls
            return
        # the swap the worker ran carries the oracle's lists
        assert self.calls[-1] == (res.request_ids, res.source_block_ids, res.target_block_ids,
                                  res.is_swap_in)
        for r in res.request_ids:
            self.table(r)                                 # same location and blocks
        ko.swap_blocks(res.source_block_ids, res.target_block_ids, res.is_swap_in,
                       self.model_gpu, self.model_cpu)
        self.counts["in" if target >= 0 else "out"] += 1

    def free(self):
        if not self.lens:
            return
        rid = int(self.rng.choice(list(self.lens)))
        # the scheduler frees a request only once its moves have finished
        for e in self.worker.move_event_table.get(rid, []):
            e.synchronize()
        self.compute.synchronize()
        self.orc.free_blocks(rid)
        self.bm.free_blocks(rid)
        self.worker.clear_request_resource(rid)
        del self.lens[rid]

    def check_pools(self):
        torch.cuda.synchronize()
        assert np.array_equal(to_bits(self.cache), self.model_gpu)
        assert np.array_equal(self.swap.view(torch.int16).numpy().view(np.uint16),
                              self.model_cpu)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_block_manager_moves_through_worker_streams(device, seed):
    run = _Run(device, seed)
    ops = ["new", "decode", "out", "in", "free"]
    p = [0.25, 0.35, 0.17, 0.15, 0.08]
    for i in range(90):
        op = ops[int(run.rng.choice(len(ops), p=p))]
        if op == "new":
            run.new_requests()
        elif op == "decode":
            run.decode()
        elif op == "out":
            run.move(CPU)
        elif op == "in":
            run.move(0)
        else:
            run.free()
        if i % 15 == 14:
            run.check_pools()
    run.check_pools()
    c = run.counts
    assert c["out"] >= 3 and c["in"] >= 3 and c["decode"] >= 10, c
