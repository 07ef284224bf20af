"""The shared swap-space file and cross-process move events on the GPU
(aegaeon/aegaeon/llm.py:297-318, worker.py:130-147,716-815,
utils.py:306-331).

* The file mapping (the reference's layout: block b of a shape at byte
  b * block_bytes, mapped shared as float16) reached through a pinned bounce
  buffer: ops.swap out of and back into the GPU pool, with bounce buffers that
  force several chunks, bit-exact against the oracle's swap; the file holds
  what a second, independent mapping of it reads.
* Two processes on the GPU sharing the file and exchanging move signals (the
  stand-in for the reference's interprocess events, whose record this HIP
  runtime refuses): the child swaps in what the parent swapped out, waiting
  on the parent's exported move while the parent's swap-out is still held
  behind a spin; then the parent swaps in what the child swapped out, waiting
  on the child's.  Both sides check the bytes against seeded data, and
  neither wait timed out.
"""
import json
import os
import queue
import subprocess
import sys
import threading
import uuid
from pathlib import Path

import numpy as np
import pytest
import torch

from aegaeon_amd import ops, swap_pool
from aegaeon_amd.worker_swap import KVSwapWorker
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent
SHAPE = (2, 2, 16, 4, 128)           # 64 KiB bf16 blocks
BB = int(np.prod(SHAPE)) * 2
N_SLABS, SLAB = 8, 4 << 20           # a 32 MiB file: 512 blocks


@pytest.fixture
def shm_path():
    p = f"/dev/shm/aegkv_test_{os.getpid()}_{uuid.uuid4().hex[:8]}"
    yield p
    try:
        os.unlink(p)
    except FileNotFoundError:
        pass


def _seeded(seed, n):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-2 ** 15, 2 ** 15, (n, *SHAPE), dtype=torch.int16, generator=g)


@pytest.mark.parametrize("bounce_blocks,staging_blocks", [(3, 5), (64, 64), (1, 1)])
def test_swap_through_file_mapping(device, shm_path, bounce_blocks, staging_blocks):
    """Swap-out into the shared file and swap-in back through bounce buffers
    of 1-64 blocks (so 1 to 40 chunks), scattered ids on both sides."""
    rng = np.random.default_rng(bounce_blocks)
    kv_swap = swap_pool.init_cpu_cache(N_SLABS, SLAB, shm_path)
    assert not kv_swap.is_pinned() and kv_swap.numel() * 2 == N_SLABS * SLAB
    n_host = kv_swap.numel() * 2 // BB
    N = 96
    bits = _seeded(3, N)
    cache = bits.view(torch.bfloat16).to(device)
    src = rng.permutation(N)[:40]
    host_ids = rng.permutation(n_host)[:40]
    back = rng.permutation(np.setdiff1d(np.arange(N), src))[:40]
    bounce = swap_pool.bounce_buffer(bounce_blocks * BB)
    staging = torch.empty(staging_blocks * BB, dtype=torch.uint8, device=device)
    ops.swap(src, host_ids, False, cache, kv_swap, staging=staging, bounce=bounce)
    ops.swap(host_ids, back, True, cache, kv_swap, staging=staging, bounce=bounce)
    torch.cuda.synchronize()
    ref_gpu = bits.numpy().view(np.uint16).copy()
    ref_host = np.zeros((n_host, *SHAPE), dtype=np.uint16)
    ko.swap_blocks(src, host_ids, False, ref_gpu, ref_host)
    ko.swap_blocks(host_ids, back, True, ref_gpu, ref_host)
    assert np.array_equal(cache.view(torch.int16).cpu().numpy().view(np.uint16), ref_gpu)
    # a second, independent mapping of the file reads the same bytes
    again = swap_pool.init_cpu_cache(N_SLABS, SLAB, shm_path)
    assert np.array_equal(again.view(torch.int16).numpy().view(np.uint16).reshape(ref_host.shape),
                          ref_host)


def test_swaps_on_two_streams_through_one_file(device, shm_path):
    """Two swap-outs into disjoint parts of the file, enqueued on two streams
    behind a held stream, then two swap-ins back on the two streams: the
    library's host-copy stream serves both calls, and its event ordering
    keeps each chunk's halves apart and each swap-in after its own stream's
    swap-out."""
    rng = np.random.default_rng(21)
    kv_swap = swap_pool.init_cpu_cache(N_SLABS, SLAB, shm_path)
    n_host = kv_swap.numel() * 2 // BB
    N = 96
    bits = _seeded(7, N)
    cache = bits.view(torch.bfloat16).to(device)
    perm = rng.permutation(N)
    src = [perm[:24], perm[24:48]]
    hperm = rng.permutation(n_host)
    host_ids = [hperm[:24], hperm[24:48]]
    back = [perm[48:72], perm[72:96]]
    streams = [torch.cuda.Stream(device), torch.cuda.Stream(device)]
    bounces = [swap_pool.bounce_buffer(4 * BB), swap_pool.bounce_buffer(5 * BB)]
    stagings = [torch.empty(3 * BB, dtype=torch.uint8, device=device) for _ in range(2)]
    torch.cuda.synchronize()
    torch.cuda._sleep(50_000_000)  # both streams start behind this hold
    held = torch.cuda.Event()
    held.record()
    for i in range(2):
        streams[i].wait_event(held)
        with torch.cuda.stream(streams[i]):
            ops.swap(src[i], host_ids[i], False, cache, kv_swap, staging=stagings[i],
                     bounce=bounces[i])
    for i in range(2):
        with torch.cuda.stream(streams[i]):
            ops.swap(host_ids[i], back[i], True, cache, kv_swap, staging=stagings[i],
                     bounce=bounces[i])
    torch.cuda.synchronize()
    ref_gpu = bits.numpy().view(np.uint16).copy()
    ref_host = np.zeros((n_host, *SHAPE), dtype=np.uint16)
    for i in range(2):
        ko.swap_blocks(src[i], host_ids[i], False, ref_gpu, ref_host)
        ko.swap_blocks(host_ids[i], back[i], True, ref_gpu, ref_host)
    assert np.array_equal(cache.view(torch.int16).cpu().numpy().view(np.uint16), ref_gpu)
    got_host = kv_swap.view(torch.int16).numpy().view(np.uint16).reshape(ref_host.shape)
    assert np.array_equal(got_host, ref_host)


def test_pageable_swap_space_needs_a_bounce_buffer(device, shm_path):
    kv_swap = swap_pool.init_cpu_cache(N_SLABS, SLAB, shm_path)
    cache = torch.zeros((4, *SHAPE), dtype=torch.bfloat16, device=device)
    with pytest.raises(ValueError):
        ops.swap([0], [0], False, cache, kv_swap)
    with pytest.raises(ValueError):   # a bounce buffer that is not pinned
        ops.swap([0], [0], False, cache, kv_swap, bounce=torch.empty(BB, dtype=torch.uint8))


def test_two_processes_share_file_and_move_events(device, shm_path):
    kv_swap = swap_pool.init_cpu_cache(N_SLABS, SLAB, shm_path)
    cache = torch.zeros((64, *SHAPE), dtype=torch.bfloat16, device=device)
    worker = KVSwapWorker(cache, kv_swap, interprocess=True, bounce_bytes=1 << 20)
    err = open(shm_path + ".child.log", "w+")
    child = subprocess.Popen([sys.executable, "-u", str(HERE / "swap_file_child.py"), shm_path,
                              str(N_SLABS), str(SLAB)],
                             stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=err,
                             text=True, cwd=str(HERE.parent))

    lines = queue.Queue()
    reader = threading.Thread(target=lambda: [lines.put(x) for x in child.stdout] + [lines.put("")],
                              daemon=True)
    reader.start()

    def recv(timeout=90.0):
        try:
            line = lines.get(timeout=timeout)
        except queue.Empty:
            child.kill()
            raise AssertionError("the child process did not answer in time")
        if not line:
            err.seek(0)
            raise AssertionError(f"child ended early: {err.read()[-2000:]}")
        return json.loads(line)

    def send(obj):
        child.stdin.write(json.dumps(obj) + "\n")
        child.stdin.flush()

    try:
        assert recv() == {"ready": True}
        hold = int(0.2 * 1.2e9)                 # ~200 ms of spin (~1.2 GHz shader clock)
        dev_ids = list(range(0, 24))
        file_ids = [int(x) for x in np.random.default_rng(4).permutation(256)[:24]]
        cache[torch.tensor(dev_ids, device=device)] = _seeded(11, 24).to(device).view(
            torch.bfloat16)
        torch.cuda.synchronize()
        with torch.cuda.stream(worker.swap_out_stream):
            torch.cuda._sleep(hold)             # the swap-out is still pending below
        ev = worker.swap_blocks([1], dev_ids, file_ids, [None], False)
        assert not ev.query()
        d, pid, raw, word, serial = worker.export(ev)
        out_file_ids = list(range(300, 316))
        send({"handle": [d, pid, raw.hex(), word, serial], "file_ids": file_ids,
              "dev_ids": list(range(40, 64)), "seed": 11, "out_file_ids": out_file_ids,
              "out_seed": 12, "hold_cycles": hold})
        reply = recv()
        assert reply["ok"], reply["detail"]
        # the child's swap-out is held behind its own spin: wait on its event
        d2, pid2, raw2, w2, s2 = reply["handle"]
        ev_in = worker.swap_blocks([8], out_file_ids, list(range(48, 64)),
                                   [(int(d2), int(pid2), bytes.fromhex(raw2), int(w2), int(s2))],
                                   True)
        ev_in.synchronize()
        worker.check_timeouts()
        got = cache[48:64].view(torch.int16).cpu()
        assert torch.equal(got, _seeded(12, 16))
        # the parent's own mapping of the file holds the child's blocks too
        host = kv_swap.view(torch.int16).view(-1, *SHAPE)
        assert torch.equal(host[out_file_ids], _seeded(12, 16))
        assert torch.equal(host[file_ids], _seeded(11, 24))
        send({"done": True})
        assert child.wait(timeout=60) == 0
    finally:
        if child.poll() is None:
            child.kill()
            child.wait()
        torch.cuda.synchronize()
        swap_pool.close_opened()
        err.close()
        os.unlink(shm_path + ".child.log")


def test_signal_array_checks_words_and_timeout_word(device):
    """Word indexes outside the array and a timeout word the wait kernel could
    not write are refused before any launch."""
    arr = swap_pool.SignalArray(4, device)
    try:
        stream = torch.cuda.current_stream(device)
        with pytest.raises(IndexError):
            arr.signal(stream, 4, 1)
        with pytest.raises(IndexError):
            swap_pool.reduce_event(arr, -1, 1)
        with pytest.raises(ValueError):
            arr.wait(stream, 0, 1, torch.zeros(1, dtype=torch.int32))  # host tensor
        with pytest.raises(ValueError):
            arr.wait(stream, 0, 1, torch.zeros(1, dtype=torch.int64, device=device))
        # a word that is already reached: the wait ends at once
        timed_out = torch.zeros(1, dtype=torch.int32, device=device)
        arr.signal(stream, 3, 5)
        arr.wait(stream, 3, 5, timed_out, timeout_s=10.0)
        torch.cuda.synchronize(device)
        assert int(timed_out.item()) == 0
    finally:
        arr.close()
    with pytest.raises(ValueError):
        arr.word(0)


def test_own_exported_handle_orders_a_later_swap(device):
    """A move handle this process exported, passed as ``after=`` (no request
    id), orders the later swap on the other stream behind the held swap-out:
    the swap-in reads what the swap-out wrote, not the stale host bytes."""
    cache = torch.zeros((16, *SHAPE), dtype=torch.bfloat16, device=device)
    host = torch.zeros((8, *SHAPE), dtype=torch.bfloat16, pin_memory=True)
    worker = KVSwapWorker(cache, host, interprocess=True)
    cache[0:4] = _seeded(21, 4).to(device).view(torch.bfloat16)
    torch.cuda.synchronize()
    with torch.cuda.stream(worker.swap_out_stream):
        torch.cuda._sleep(int(0.05 * 1.2e9))     # ~50 ms: the swap-out is pending below
    ev = worker.swap_blocks([1], [0, 1, 2, 3], [4, 5, 6, 7], [None], False)
    assert not ev.query()
    handle = worker.export(ev)
    ev_in = worker.swap_blocks([2], [4, 5, 6, 7], [8, 9, 10, 11], [None], True, after=[handle])
    ev_in.synchronize()
    worker.wait_for_all_move_out()
    assert torch.equal(cache[8:12].view(torch.int16).cpu(), _seeded(21, 4))
    assert swap_pool.query_event(handle)
    worker.signals.close()


def test_cross_process_wait_timeout_raises_at_host_sync_points(device):
    """A wait on a move that never completes gives up after its bound (set
    tiny here, so the wait kernel ends at once) and the next host point that
    treats moves as complete raises instead of letting the unordered work
    pass silently."""
    cache = torch.zeros((8, *SHAPE), dtype=torch.bfloat16, device=device)
    host = torch.zeros((8, *SHAPE), dtype=torch.bfloat16, pin_memory=True)
    worker = KVSwapWorker(cache, host, wait_timeout_s=1e-3)
    arr = swap_pool.SignalArray(2, device)
    try:
        never = swap_pool.reduce_event(arr, 1, 7)   # word 1 is never set
        assert not swap_pool.query_event(never)
        worker.swap_blocks([3], [0], [1], [None], True, after=[never])
        with pytest.raises(TimeoutError):
            worker.wait_for_all_move_in()
        with pytest.raises(TimeoutError):
            worker.ready_mask([3])
        arr.signal(torch.cuda.current_stream(device), 1, 7)
        torch.cuda.synchronize(device)
        assert swap_pool.query_event(never) and arr.read(1) == 7
    finally:
        torch.cuda.synchronize(device)
        arr.close()


def test_block_manager_reclaim_polls_exported_handles(device):
    """The block manager's reclaim polls interprocess move handles from the
    host (``query_event``), without blocking the event loop, and reclaims
    the source blocks once the held swap-out is done."""
    import asyncio
    from aegaeon_amd.block_manager import BLOCK_LOCATION_CPU, BlockManager
    cache = torch.zeros((8, *SHAPE), dtype=torch.bfloat16, device=device)
    host = torch.zeros((16, *SHAPE), dtype=torch.bfloat16, pin_memory=True)
    worker = KVSwapWorker(cache, host, interprocess=True)
    remote = worker.remote_callable()

    def exporting(method, *args):
        out = remote(method, *args)
        return worker.export(out) if method == "swap_blocks" else out

    bm = BlockManager(1, 16 * BB)
    bm.register_gpu_space(0, 8, SHAPE, exporting)

    class R:
        def __init__(self, rid, n):
            self.request_id, self.n, self.is_finished = rid, n, False

        def get_input_len(self):
            return self.n

        def get_output_len(self):
            return 0

    r1 = R(1, 16 * 6)
    asyncio.run(bm.allocate_blocks_batched([r1], 0))
    with torch.cuda.stream(worker.swap_out_stream):
        torch.cuda._sleep(int(0.05 * 1.2e9))
    asyncio.run(bm.move_requests([r1], BLOCK_LOCATION_CPU))
    ticks = []

    async def other():
        for _ in range(3):
            ticks.append(1)
            await asyncio.sleep(0.001)

    async def main():
        await asyncio.gather(bm.allocate_blocks_batched([R(2, 16 * 4)], 0), other())

    asyncio.run(main())
    assert len(ticks) == 3
    assert bm.get_block_table(2).blocks == [6, 7, 0, 1]
    torch.cuda.synchronize(device)
    worker.signals.close()
