"""Benchmark of the MI355X KV-cache data path (one GPU).

Headline (``value``): KV append throughput in GB/s for the Qwen2.5-7B-shaped
decode step (28 layers, 4 KV heads, D 128, bf16, block 16, 256 sequences with
context lengths lognormal(mean 600, sigma 1) clipped to [16, 4096], pool = 2x
the need, scattered block tables), all layers in one launch.  A "step" is one
such append.  Algorithmic bytes per step: read K and V, write them into the
paged pool, read the slot mapping: ``2 * B * L * 2 * Hkv * D * 2 + 8 * B``.

The timed steps rotate over 32 successive decode steps (distinct K/V inputs and
slot mappings, ~0.9 GB of distinct traffic), so the 256 MB last-level cache
cannot serve the inputs from a previous step: every step reads and writes HBM.

Timing.  The host enqueues a launch in ~10 us of Python; a 8 us kernel would
then measure the host.  Each timed region therefore starts behind a bounded
spin kernel (torch.cuda._sleep) that holds the stream while the host enqueues
all K launches; the GPU then runs them back to back.  HIP events recorded on
the stream the kernels run on (torch's current stream, which every op of the
package launches on) bracket the K launches; their elapsed time over K is the
average device duration of one step, the quantity rocprofv3 reports per
kernel (back-to-back launches leave no gap between kernels).  ``value`` and
``roofline.achieved`` are the algorithmic bytes over that duration.
torch.cuda.synchronize() brackets every timed region.

Secondary lines (``ops``): the per-layer launch pattern of vLLM; paged decode
attention (Qwen2.5-7B GQA 28/4, 128 sequences, lognormal mean 1500, up to 8192
tokens) in us per layer; block pack and scatter for the Llama-2-13B swap
workload (32 x 2048 tokens, 4096 blocks of 12.5 MiB) and the same swap through
ops.swap out to pinned host memory and back (all 4096 blocks when the host can
pin them), with its pack, DMA and scatter legs; defrag of the unified
multi-model pool followed by a Yi-1.5-9B
decode step (append + attention); token gather; a swap-out on a side stream
overlapped with 28 layers of decode attention; the prefill side (prompt KV
write and causal varlen attention, 4 x 2048 tokens); device-side input preparation
against the reference's host loops; the block manager's host bookkeeping
(native against the reference's algorithm, same block ids); the copy floor,
the block-copy kernel moving the headline append's bytes.

The CPU baseline is the reference's path restated with torch on the host
(oracle/torch_cpu.py) on every core of the affinity mask, 3 warm-ups and the
median of at least 10 runs: the same append into the full pool, plus one
layer of the attention batch in float32 and the swap as host memcpy.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
PCIE_PEAK_GBS = 64.0   # PCIe 5.0 x16, one direction
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense
METRIC = "KV gather/append GB/s (%HBM peak); paged decode-attn µs/layer @Qwen2.5-7B"
ROTATE_STEPS = 32


def log(msg: str) -> None:
    print(f"# {msg}", file=sys.stderr, flush=True)


class Timer:
    """Device timing of back-to-back launches on torch's current stream."""

    def __init__(self):
        import torch
        self.torch = torch
        self.cycles_per_ms = self._calibrate()

    def _calibrate(self) -> float:
        torch = self.torch
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        torch.cuda._sleep(2_000_000)
        e1.record()
        e1.synchronize()
        return 2_000_000 / max(e0.elapsed_time(e1), 1e-3)

    def _hold(self, fn, steps: int) -> None:
        """Enqueue a spin long enough to cover the host enqueue of `steps` calls."""
        torch = self.torch
        t0 = time.perf_counter()
        for i in range(3):
            fn(i)
        torch.cuda.synchronize()
        host_ms = (time.perf_counter() - t0) / 3 * 1e3
        hold_ms = min(2000.0, 2.0 * host_ms * steps + 2.0)
        torch.cuda._sleep(int(hold_ms * self.cycles_per_ms))

    def run(self, fn, steps: int):
        """Returns (device ms per call over the held region, wall s)."""
        torch = self.torch
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        self._hold(fn, steps)
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for i in range(steps):
            fn(i)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / steps, time.perf_counter() - t0


# ----------------------------------------------------------------------------- append
def bench_append(args, timer):
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd.workloads import qwen_append_batch, successive_step_slots
    dev = torch.device("cuda", 0)
    wb = qwen_append_batch(args.seed)
    g = wb.geometry
    cache = torch.empty((wb.n_pool_blocks, *g.block_shape), dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(args.seed)
    R = ROTATE_STEPS
    keys = torch.randn((R, g.n_layers, wb.batch, g.n_kv_heads, g.head_dim), generator=gen,
                       device=dev).to(torch.bfloat16)
    vals = torch.randn(keys.shape, generator=gen, device=dev).to(torch.bfloat16)
    slots = torch.from_numpy(successive_step_slots(wb, R)).to(dev)

    def cold(i):
        r = i % R
        A.append_kv(keys[r], vals[r], cache, slots[r])

    def hot(i):
        A.append_kv(keys[0], vals[0], cache, slots[0])

    view = cache.permute(1, 2, 0, 3, 4, 5)

    def per_layer(i):
        r = i % R
        for layer in range(g.n_layers):
            A.reshape_and_cache_flash(keys[r, layer], vals[r, layer], view[layer, 0],
                                      view[layer, 1], slots[r])

    for i in range(args.warmup):
        cold(i)
    torch.cuda.synchronize()
    region_ms, wall = timer.run(cold, args.steps)
    hot_ms, _ = timer.run(hot, args.steps)
    pl_ms, _ = timer.run(per_layer, max(4, args.steps // 8))
    nbytes = wb.append_bytes()
    del cache, keys, vals
    torch.cuda.empty_cache()
    return {"wb": wb, "bytes": nbytes, "ms": region_ms, "wall_s": wall, "hot_ms": hot_ms,
            "per_layer_step_ms": pl_ms}


# -------------------------------------------------------------------------- attention
def _fill_random(t, gen, chunk_blocks=1024):
    import torch
    for i in range(0, t.size(0), chunk_blocks):
        sl = t[i:i + chunk_blocks]
        sl.copy_(torch.randn(sl.shape, generator=gen, device=t.device, dtype=torch.float32)
                 .to(t.dtype))


def bench_attention(args, timer, wb=None, label="Qwen2.5-7B"):
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd.workloads import qwen_attention_batch
    dev = torch.device("cuda", 0)
    wb = wb or qwen_attention_batch(args.seed)
    g = wb.geometry
    N = wb.n_pool_blocks
    cache = torch.empty((N, *g.block_shape), dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 1)
    _fill_random(cache, gen)
    q = torch.randn((g.n_layers, wb.batch, g.n_q_heads, g.head_dim), generator=gen,
                    device=dev).to(torch.bfloat16)
    bt = torch.from_numpy(wb.padded_tables()).to(dev)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(dev)
    max_len = int(wb.seq_lens.max())
    view = cache.permute(1, 2, 0, 3, 4, 5)
    scale = 1.0 / math.sqrt(g.head_dim)
    outs = torch.empty_like(q)
    ws = A.attention_workspace(wb.batch, g.n_q_heads, g.n_kv_heads, g.head_dim, max_len,
                               torch.bfloat16, args.nwg, device=dev)

    def layer_call(i):
        layer = i % g.n_layers
        A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], bt, sl, scale,
                                 max_len, out=outs[layer], n_workgroups=args.nwg,
                                 workspace=ws)

    # A decode step: the plan of the step's tables is built at its first layer
    # (the plan build is inside the timed region, shared by the 28 layers).
    plan = [None]

    def planned_call(i):
        layer = i % g.n_layers
        if layer == 0:
            plan[0] = A.DecodePlan(bt, sl, max_len, g.n_kv_heads, args.nwg)
        A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], None, None, scale,
                                 max_len, out=outs[layer], n_workgroups=args.nwg,
                                 workspace=ws, plan=plan[0])

    # vLLM's per-layer call (flash_attn_with_kvcache), as the backend makes it:
    # every layer of a step passes the step's metadata tensors, which are new
    # at each step (here: a fresh lengths tensor at layer 0), so the call plans
    # at the step's first layer and reuses the plan in the others
    step_lens = [sl]
    q4 = q.view(g.n_layers, wb.batch, 1, g.n_q_heads, g.head_dim)
    outs4 = outs.view(g.n_layers, wb.batch, 1, g.n_q_heads, g.head_dim)

    def kvcache_call(i):
        layer = i % g.n_layers
        if layer == 0:
            step_lens[0] = sl.clone()
        A.flash_attn_with_kvcache(q4[layer], view[layer, 0], view[layer, 1],
                                  cache_seqlens=step_lens[0], block_table=bt,
                                  softmax_scale=scale, max_seqlen=max_len, out=outs4[layer])

    # The decode step as a layer runs it: the new token's K/V appended, then
    # attention over seq_len tokens (the new one included).  Two launches per
    # layer as vLLM does (reshape_and_cache_flash, then the attention), or
    # the fused call (the append inside the attention's launches).
    knew = torch.randn((g.n_layers, wb.batch, g.n_kv_heads, g.head_dim), generator=gen,
                       device=dev).to(torch.bfloat16)
    vnew = torch.randn(knew.shape, generator=gen, device=dev).to(torch.bfloat16)
    slots = torch.from_numpy(wb.slot_mapping()).to(dev)

    def two_launch_call(i):
        layer = i % g.n_layers
        if layer == 0:
            plan[0] = A.DecodePlan(bt, sl, max_len, g.n_kv_heads, args.nwg)
        A.reshape_and_cache_flash(knew[layer], vnew[layer], view[layer, 0], view[layer, 1], slots)
        A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], None, None, scale,
                                 max_len, out=outs[layer], n_workgroups=args.nwg,
                                 workspace=ws, plan=plan[0])

    def fused_call(i):
        layer = i % g.n_layers
        if layer == 0:
            plan[0] = A.DecodePlan(bt, sl, max_len, g.n_kv_heads, args.nwg)
        A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], None, None, scale,
                                 max_len, out=outs[layer], n_workgroups=args.nwg,
                                 workspace=ws, plan=plan[0], key=knew[layer],
                                 value=vnew[layer])

    for i in range(g.n_layers):
        layer_call(i)
    torch.cuda.synchronize()
    unplanned_out = outs.clone()
    for i in range(g.n_layers):
        planned_call(i)
    torch.cuda.synchronize()
    if not torch.equal(outs, unplanned_out):
        raise RuntimeError("planned and unplanned attention disagree")
    for i in range(g.n_layers):
        kvcache_call(i)
    torch.cuda.synchronize()
    if not torch.equal(outs, unplanned_out):
        raise RuntimeError("flash_attn_with_kvcache and the unplanned attention disagree")
    for i in range(g.n_layers):
        two_launch_call(i)
    torch.cuda.synchronize()
    two_out = outs.clone()
    for i in range(g.n_layers):
        fused_call(i)
    torch.cuda.synchronize()
    if not torch.equal(outs, two_out):
        raise RuntimeError("fused and two-launch append + attention disagree")
    del unplanned_out, two_out
    steps = max(g.n_layers, (args.steps // g.n_layers) * g.n_layers)
    # the five forms alternate over seven rounds and each keeps its best round,
    # so that a slow stretch of the box does not fall on one form only
    best = {}
    for _ in range(7):
        for name, fn in (("unplanned", layer_call), ("planned", planned_call),
                         ("kvcache", kvcache_call), ("two", two_launch_call),
                         ("fused", fused_call)):
            ms, _ = timer.run(fn, steps)
            best[name] = min(best.get(name, ms), ms)
    unplanned_ms, region_ms, two_ms, fused_ms = (best[k] for k in
                                                 ("unplanned", "planned", "two", "fused"))
    nbytes = wb.attention_bytes()
    del cache
    torch.cuda.empty_cache()
    return {"label": label, "wb": wb, "bytes_per_layer": nbytes, "us_per_layer": region_ms * 1e3,
            "unplanned_us_per_layer": unplanned_ms * 1e3, "two_launch_us": two_ms * 1e3,
            "fused_us": fused_ms * 1e3, "kvcache_us": best["kvcache"] * 1e3}


# ------------------------------------------------------------------------ pack / swap
def bench_pack(args, timer):
    """Llama-2-13B: pack the 4096 scattered blocks into a contiguous device
    staging buffer, scatter them into a disjoint free set; sampled PCIe leg."""
    import torch
    from aegaeon_amd import ops
    from aegaeon_amd.workloads import llama_swap_workload
    dev = torch.device("cuda", 0)
    wl = llama_swap_workload(args.seed, n_seqs=args.swap_seqs)
    g = wl.geometry
    bb = g.block_bytes
    pool = torch.empty((wl.n_pool_blocks, bb), dtype=torch.uint8, device=dev)
    pool.view(torch.int32).fill_(0x3C003C00)
    staging = torch.empty((wl.n_blocks, bb), dtype=torch.uint8, device=dev)
    src = np.asarray(wl.gpu_ids, dtype=np.int64)
    dst = np.asarray(wl.swap_in_ids, dtype=np.int64)

    def pack(i):
        ops.pack_blocks(pool, src, out=staging)

    def scatter(i):
        ops.scatter_blocks(staging, dst, pool)

    src_dev = torch.from_numpy(src).to(dev)
    dst_dev = torch.from_numpy(dst).to(dev)

    def torch_pack(i):  # the library baseline at the same bytes: index_select
        torch.index_select(pool, 0, src_dev, out=staging)

    def torch_scatter(i):
        pool.index_copy_(0, dst_dev, staging)

    # the same bytes without id lists: the pool's first blocks copied to the
    # staging buffer as one contiguous range (the ceiling of a read + write
    # stream of this size, against which the id-addressed sides are read)
    front = pool[:wl.n_blocks]

    def contig(i):
        ops.copy_blocks(front, staging, None, None)

    pack(0)
    scatter(0)
    contig(0)
    torch.cuda.synchronize()
    steps = max(2, args.steps // 40)
    p_ms, _ = timer.run(pack, steps)
    s_ms, _ = timer.run(scatter, steps)
    c_ms, _ = timer.run(contig, steps)
    tp_ms, _ = timer.run(torch_pack, steps)
    ts_ms, _ = timer.run(torch_scatter, max(1, steps // 4))
    nbytes = wl.pack_bytes()
    swap = bench_swap_host(args, wl, pool, staging, src, dst) if args.swap_blocks != 0 else None
    del pool, staging
    torch.cuda.empty_cache()
    return {"wl": wl, "bytes": nbytes, "pack_ms": p_ms, "scatter_ms": s_ms, "swap": swap,
            "torch_pack_ms": tp_ms, "torch_scatter_ms": ts_ms, "contig_ms": c_ms,
            "contig_bytes": 2 * wl.n_blocks * bb}


def bench_swap_host(args, wl, pool, staging, src, dst):
    """The Llama-2-13B swap as the worker runs it (worker.py:753-762): n of
    the 4096 scattered blocks out to a pinned host pool with ops.swap (staged:
    pack into a 256 MiB device buffer, one DMA per run of host ids) and back
    into the disjoint free set with ops.swap (DMA into staging, scatter).  n is
    4096 when the host can pin the 50 GiB (64 GiB after torch's power-of-two
    rounding), else the largest power-of-two fraction that fits; the line
    states n.  The DMA legs alone are ops.swap of the contiguous staging
    buffer (no pack: one DMA for all n blocks each way).  Each figure is the
    median of 3 calls, timed with events on the calling stream."""
    import torch
    from aegaeon_amd import ops
    from aegaeon_amd.workloads import pinnable_blocks
    bb = wl.geometry.block_bytes
    want = wl.n_blocks if args.swap_blocks < 0 else min(args.swap_blocks, wl.n_blocks)
    n = pinnable_blocks(bb, want)
    if n == 0:
        return None
    t0 = time.perf_counter()
    host = torch.empty((n, bb), dtype=torch.uint8, pin_memory=True)
    pin_s = time.perf_counter() - t0
    host_ids = np.arange(n, dtype=np.int64)

    def timed(fn, reps=3):
        out = []
        for _ in range(reps):
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            fn()
            e1.record()
            torch.cuda.synchronize()
            out.append(e0.elapsed_time(e1))
        return sorted(out)[len(out) // 2]

    res = {"blocks": n, "of_blocks": wl.n_blocks, "pin_s": pin_s}
    res["swap_out_ms"] = timed(lambda: ops.swap(src[:n], host_ids, False, pool, host))
    res["swap_in_ms"] = timed(lambda: ops.swap(host_ids, dst[:n], True, pool, host))
    res["dma_d2h_ms"] = timed(lambda: ops.swap(host_ids, host_ids, False, staging[:n], host,
                                               staging=None))
    res["dma_h2d_ms"] = timed(lambda: ops.swap(host_ids, host_ids, True, staging[:n], host,
                                               staging=None))
    res["pack_ms"] = timed(lambda: ops.pack_blocks(pool, src[:n], out=staging[:n]))
    res["scatter_ms"] = timed(lambda: ops.scatter_blocks(staging[:n], dst[:n], pool))
    # the reference's shared swap file, reached through a pinned bounce buffer
    # (the file cannot be page-locked here): the same swap for a sample
    res["file"] = bench_swap_file(pool, src, dst, bb, min(n, FILE_SWAP_BLOCKS), timed)
    # the round trip is bit-exact (checked here on a sample; the tests check all)
    k = torch.from_numpy(src[:min(n, 8)]).to(pool.device)
    j = torch.from_numpy(dst[:min(n, 8)]).to(pool.device)
    ops.swap(src[:n], host_ids, False, pool, host)
    ops.swap(host_ids, dst[:n], True, pool, host)
    torch.cuda.synchronize()
    if not torch.equal(pool[k], pool[j]) or not torch.equal(host[:len(k)].to(pool.device),
                                                             pool[k]):
        raise RuntimeError("swap round trip is not bit-exact")
    del host
    torch._C._host_emptyCache()
    return res


FILE_SWAP_BLOCKS = 256          # 3.2 GiB of Llama-2-13B blocks in /dev/shm


def bench_swap_file(pool, src, dst, bb, n, timed):
    """ops.swap out to and back from a /dev/shm file of n blocks (the
    reference's swap-space file, llm.py:297-318) through a 256 MiB pinned
    bounce buffer, against the same call into pinned memory."""
    import torch
    import uuid
    from aegaeon_amd import ops, swap_pool
    path = f"/dev/shm/aegkv_bench_{os.getpid()}_{uuid.uuid4().hex[:6]}"
    try:
        kv_swap = swap_pool.init_cpu_cache(1, n * bb, path)
        bounce = swap_pool.bounce_buffer(256 << 20)
        ids = np.arange(n, dtype=np.int64)
        out = {"blocks": n,
               "swap_out_ms": timed(lambda: ops.swap(src[:n], ids, False, pool, kv_swap,
                                                     bounce=bounce)),
               "swap_in_ms": timed(lambda: ops.swap(ids, dst[:n], True, pool, kv_swap,
                                                    bounce=bounce))}
        k = torch.from_numpy(src[:4]).to(pool.device)
        j = torch.from_numpy(dst[:4]).to(pool.device)
        torch.cuda.synchronize()
        if not torch.equal(pool[k], pool[j]):
            raise RuntimeError("swap through the file is not bit-exact")
        del kv_swap, bounce
        return out
    finally:
        try:
            os.unlink(path)
        except FileNotFoundError:
            pass


# ------------------------------------------------------------- unified pool + defrag
def bench_defrag(args, timer):
    """Unified pool co-hosting Yi-1.5-9B, Qwen2.5-7B and Llama-2-13B blocks in
    1 GiB slabs at 50% occupancy: compact each model's live blocks into the
    dense prefix of its id space, then one Yi decode step (append + attention)
    through the rewritten tables."""
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd import ops
    from aegaeon_amd.pool import plan_compaction, remap_tables
    from aegaeon_amd.workloads import DecodeBatch, unified_pool_workload
    dev = torch.device("cuda", 0)
    wl = unified_pool_workload(args.seed)
    pool = torch.empty(wl.pool_bytes, dtype=torch.uint8, device=dev)
    pool.view(torch.int32).fill_(0x3F803F80)
    moved_bytes, ms, plans = 0, 0.0, {}
    for name, g in wl.geometries.items():
        live = [b for t in wl.tables[name] for b in t]
        src, dst = plan_compaction(live, wl.valid_ids(name))
        plans[name] = (src, dst)
    # time the three shape-wise compactions as one step (they touch disjoint slabs)
    snapshot = {n: (np.asarray(s), np.asarray(d)) for n, (s, d) in plans.items()}

    def defrag(i):
        for name, (s, d) in snapshot.items():
            if len(s):
                # forward on even steps, back on odd ones, so every step moves bytes
                a, b = (s, d) if i % 2 == 0 else (d, s)
                ops.defrag_blocks(pool, a, b, block_bytes=wl.geometries[name].block_bytes)

    # the library baseline at the same bytes: per shape, index_select of the
    # live blocks above the prefix into a temporary, then index_copy_ into the
    # holes (torch offers no in-place gather-scatter of disjoint rows)
    views = {}
    for name, (s, d) in snapshot.items():
        bb = wl.geometries[name].block_bytes
        nb = wl.pool_bytes // bb
        views[name] = (pool[:nb * bb].view(nb, bb), torch.from_numpy(s).to(dev),
                       torch.from_numpy(d).to(dev))

    def torch_defrag(i):
        for name, (v, s, d) in views.items():
            if s.numel():
                a, b = (s, d) if i % 2 == 0 else (d, s)
                v.index_copy_(0, b, torch.index_select(v, 0, a))

    defrag(0)
    defrag(1)
    torch_defrag(0)
    torch_defrag(1)
    torch.cuda.synchronize()
    steps = max(2, args.steps // 20)
    defrag_ms, _ = timer.run(defrag, steps)
    torch_defrag_ms, _ = timer.run(torch_defrag, 2)
    del views
    for name, (s, d) in snapshot.items():
        moved_bytes += 2 * len(s) * wl.geometries[name].block_bytes + 16 * len(s)
    n_moved = {n: int(len(s)) for n, (s, _) in snapshot.items()}

    # Yi decode step through the compacted tables, on the same byte pool
    g = wl.geometries[wl.decode_model]
    src, dst = plans[wl.decode_model]
    tables = remap_tables(wl.tables[wl.decode_model], src, dst)
    nb = wl.pool_bytes // g.block_bytes
    typed = pool[:nb * g.block_bytes].view(torch.bfloat16).view(nb, *g.block_shape)
    ctx = wl.yi_context_lens
    wb = DecodeBatch(g, ctx, tables, nb, args.seed)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 2)
    key = torch.randn((g.n_layers, wb.batch, g.n_kv_heads, g.head_dim), generator=gen,
                      device=dev).to(torch.bfloat16)
    val = torch.randn(key.shape, generator=gen, device=dev).to(torch.bfloat16)
    slots = torch.from_numpy(wb.slot_mapping()).to(dev)
    q = torch.randn((g.n_layers, wb.batch, g.n_q_heads, g.head_dim), generator=gen,
                    device=dev).to(torch.bfloat16)
    bt = torch.from_numpy(wb.padded_tables()).to(dev)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(dev)
    max_len = int(wb.seq_lens.max())
    view = typed.permute(1, 2, 0, 3, 4, 5)
    out = torch.empty_like(q)
    ws = A.attention_workspace(wb.batch, g.n_q_heads, g.n_kv_heads, g.head_dim, max_len,
                               torch.bfloat16, args.nwg, device=dev)
    scale = 1.0 / math.sqrt(g.head_dim)

    def app(i):
        A.append_kv(key, val, typed, slots)

    plan = [None]

    def attn(i):  # one decode plan per step of 48 layers, its build included
        layer = i % g.n_layers
        if layer == 0:
            plan[0] = A.DecodePlan(bt, sl, max_len, g.n_kv_heads, args.nwg)
        A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], None, None, scale,
                                 max_len, out=out[layer], n_workgroups=args.nwg,
                                 workspace=ws, plan=plan[0])

    app(0)
    attn(0)
    torch.cuda.synchronize()
    a_ms, _ = timer.run(app, max(4, args.steps // 4))
    t_ms, _ = timer.run(attn, g.n_layers * max(1, args.steps // 100))
    del pool, typed
    torch.cuda.empty_cache()
    return {"defrag_ms": defrag_ms, "torch_defrag_ms": torch_defrag_ms,
            "defrag_bytes": moved_bytes, "moved_blocks": n_moved,
            "yi_append_ms": a_ms, "yi_append_bytes": wb.append_bytes(),
            "yi_attn_us_per_layer": t_ms * 1e3, "yi_attn_bytes": wb.attention_bytes(),
            "yi_batch": wb.batch}


# --------------------------------------------------------------------------- gather
def bench_gather(args, timer):
    """De-page every sequence of the Qwen2.5-7B append batch (one layer, K and
    V) into contiguous [sum(len), Hkv, D] buffers."""
    import torch
    from aegaeon_amd import attention as A, ops
    from aegaeon_amd.workloads import qwen_append_batch
    dev = torch.device("cuda", 0)
    wb = qwen_append_batch(args.seed)
    g = wb.geometry
    cache = torch.empty((wb.n_pool_blocks, *g.block_shape), dtype=torch.bfloat16, device=dev)
    cache.view(torch.int16).fill_(0x3F80)
    bt = torch.from_numpy(wb.padded_tables()).to(dev)
    sl_np = wb.seq_lens
    sl = torch.from_numpy(sl_np.astype(np.int32)).to(dev)
    total, max_len = int(sl_np.sum()), int(sl_np.max())
    # the sequences' start rows, as the step's input preparation provides them
    cu = torch.tensor(np.concatenate([[0], np.cumsum(sl_np)]), dtype=torch.int32, device=dev)
    outs = {}

    def gather(i):
        layer = i % g.n_layers
        outs[0] = A.gather_tokens(cache, bt, sl, total, max_len, layers=(layer, 1), cu_seqlens=cu)

    # the library baseline: torch index_select of the same sequences' whole
    # blocks (16 rows each, the last ones partly past the sequence) of one
    # layer's K and V view
    view = cache.permute(1, 2, 0, 3, 4, 5)
    flat_ids = torch.from_numpy(np.concatenate(
        [np.asarray(t, dtype=np.int64) for t in wb.block_tables])).to(dev)
    n_blk = int(flat_ids.numel())
    tk = torch.empty((n_blk, *view.shape[3:]), dtype=cache.dtype, device=dev)
    tv = torch.empty_like(tk)

    def torch_gather(i):
        layer = i % g.n_layers
        torch.index_select(view[layer, 0], 0, flat_ids, out=tk)
        torch.index_select(view[layer, 1], 0, flat_ids, out=tv)

    # the same rows without a table: one contiguous range of the pool copied
    # to a buffer of the gather's output size (a read + write stream of the
    # same bytes)
    row_bytes = 2 * total * g.row_elems * 2
    flat = cache.view(torch.uint8).view(-1)[:row_bytes].view(1, row_bytes)
    flat_out = torch.empty_like(flat)

    def contig(i):
        ops.copy_blocks(flat, flat_out, None, None, block_bytes=row_bytes)

    gather(0)
    torch_gather(0)
    contig(0)
    torch.cuda.synchronize()
    region_ms, _ = timer.run(gather, max(g.n_layers, args.steps // 4))
    torch_ms, _ = timer.run(torch_gather, max(g.n_layers, args.steps // 8))
    contig_ms, _ = timer.run(contig, max(g.n_layers, args.steps // 4))
    torch_bytes = 2 * 2 * n_blk * 16 * g.row_elems * 2
    nbytes = 2 * 2 * total * g.row_elems * 2 + 4 * sum(-(-int(x) // 16) for x in sl_np)
    del cache, tk, tv, flat_out
    torch.cuda.empty_cache()
    return {"bytes": nbytes, "ms": region_ms, "torch_ms": torch_ms, "torch_bytes": torch_bytes,
            "contig_ms": contig_ms, "contig_bytes": 2 * row_bytes}


# ------------------------------------------------------------- input preparation
def bench_prepare(args, timer):
    """Per-step metadata (slot mapping, padded tables, lengths, start offsets)
    for the Qwen2.5-7B decode batch (256 requests) and a prefill batch (8
    prompts of 2048 tokens): the library's one upload + one kernel, fed from the
    reference's request lists or from arrays (the block manager's flat tables),
    against the reference's host loops (the oracle's restatement of
    worker.py:596-676) followed by the reference's eight host-to-device
    tensors.  Wall time per step, synchronised, host work included."""
    import torch
    from aegaeon_amd import inputs as I
    from aegaeon_amd.workloads import qwen_append_batch
    from oracle import kv_oracle as ko
    dev = torch.device("cuda", 0)
    wb = qwen_append_batch(args.seed)
    rng = np.random.default_rng(args.seed)
    perm = iter(rng.permutation(8 * 128).tolist())
    pre_tables = [[next(perm) for _ in range(128)] for _ in range(8)]
    pre_reqs = [(i, rng.integers(0, 32000, 2048).tolist(), 2048, 0) for i in range(8)]
    cases = {"qwen_decode_256": (I.decode_requests(wb.context_lens), wb.block_tables),
             "prefill_8x2048": (pre_reqs, pre_tables)}
    out = {}

    def reference_path(reqs, tables):
        r = ko.prepare_model_inputs(reqs, tables)
        for k in ("input_tokens", "input_positions", "slot_mapping", "block_tables",
                  "seq_lens_tensor", "context_lens_tensor", "query_start_loc", "seq_start_loc"):
            torch.from_numpy(np.ascontiguousarray(r[k])).to(dev)

    for name, (reqs, tables) in cases.items():
        times = {}
        # the same batch as arrays (the block manager's flat_block_tables layout)
        offs = np.concatenate([[0], np.cumsum([len(t) for t in tables])]).astype(np.int64)
        ids = np.concatenate([np.asarray(t, dtype=np.int32) for t in tables])
        seq = np.asarray([r[2] for r in reqs], dtype=np.int32)
        ctx = np.asarray([r[3] for r in reqs], dtype=np.int32)
        toks = np.concatenate([np.asarray(r[1], dtype=np.int64) for r in reqs])
        for label, fn in (("device", lambda: I.prepare_model_inputs(reqs, tables, dev)),
                          ("device_from_arrays",
                           lambda: I.prepare_inputs_from_arrays(ids, offs, seq, ctx, toks, dev)),
                          ("reference_host", lambda: reference_path(reqs, tables))):
            for _ in range(3):
                fn()
            torch.cuda.synchronize()
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 0.5 or n < 5:
                fn()
                torch.cuda.synchronize()
                n += 1
            times[label] = (time.perf_counter() - t0) / n * 1e6
        out[name] = times
    return out


# ------------------------------------------------------------------------- overlap
OVERLAP_SWAP_BLOCKS = 128   # 112 MiB of Qwen2.5-7B blocks


def bench_overlap(args, timer):
    """Swap-out on a side stream overlapped with compute: 28 layers of the
    Qwen2.5-7B decode attention (128 sequences) on the compute stream while
    128 scattered Qwen2.5-7B blocks (112 MiB) are swapped out to pinned host
    memory on a second stream, as the reference's worker does with its swap
    streams (worker.py:716-770).  Both streams are held behind a spin until
    the host has enqueued everything; events give each stream's span."""
    import torch
    from aegaeon_amd import attention as A, ops
    from aegaeon_amd.workloads import qwen_attention_batch
    dev = torch.device("cuda", 0)
    wb = qwen_attention_batch(args.seed)
    g = wb.geometry
    cache = torch.empty((wb.n_pool_blocks, *g.block_shape), dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 3)
    _fill_random(cache, gen)
    view = cache.permute(1, 2, 0, 3, 4, 5)
    q = torch.randn((g.n_layers, wb.batch, g.n_q_heads, g.head_dim), generator=gen,
                    device=dev).to(torch.bfloat16)
    outs = torch.empty_like(q)
    bt = torch.from_numpy(wb.padded_tables()).to(dev)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(dev)
    max_len = int(wb.seq_lens.max())
    scale = 1.0 / math.sqrt(g.head_dim)
    ws = A.attention_workspace(wb.batch, g.n_q_heads, g.n_kv_heads, g.head_dim, max_len,
                               torch.bfloat16, 0, device=dev)
    rng = np.random.default_rng(args.seed + 3)
    src = rng.choice(wb.n_pool_blocks, OVERLAP_SWAP_BLOCKS, replace=False).astype(np.int64)
    dst = np.arange(OVERLAP_SWAP_BLOCKS, dtype=np.int64)
    host = torch.empty((OVERLAP_SWAP_BLOCKS, *g.block_shape), dtype=torch.bfloat16,
                       pin_memory=True)
    main = torch.cuda.current_stream(dev)
    side = torch.cuda.Stream(device=dev)

    def attn_all():
        for layer in range(g.n_layers):
            A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], bt, sl, scale,
                                     max_len, out=outs[layer], workspace=ws)

    def swap_out():
        with torch.cuda.stream(side):
            ops.swap(src, dst, False, cache, host)

    def span(run_attn: bool, run_swap: bool) -> float:
        ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
        torch.cuda.synchronize()
        torch.cuda._sleep(int(20.0 * timer.cycles_per_ms))  # hold both streams
        gate, e0, e_side, e_end = ev(), ev(), ev(), ev()
        gate.record(main)
        side.wait_event(gate)
        e0.record(main)
        if run_swap:
            swap_out()
        e_side.record(side)
        if run_attn:
            attn_all()
        main.wait_event(e_side)
        e_end.record(main)
        torch.cuda.synchronize()
        return e0.elapsed_time(e_end)

    attn_all()
    swap_out()
    torch.cuda.synchronize()
    reps = 3
    t_a = sorted(span(True, False) for _ in range(reps))[reps // 2]
    t_s = sorted(span(False, True) for _ in range(reps))[reps // 2]
    t_b = sorted(span(True, True) for _ in range(reps))[reps // 2]
    del cache, q, outs, host
    torch.cuda.empty_cache()
    return {"attn_ms": t_a, "swap_ms": t_s, "both_ms": t_b,
            "swap_bytes": OVERLAP_SWAP_BLOCKS * g.block_bytes}


# ------------------------------------------------------------------------- prefill
PREFILL_LENS = [2048] * 4   # the reference's profiled prefill shape i2048b4
PREFILL_LONG = 8192         # one long prompt: the attention kernel's steady state
PREFILL_RAGGED = [1700, 300, 2048, 77, 1024, 640, 129, 2000]  # a mixed prompt batch


def bench_prefill(args, timer):
    """Prompt run of a Qwen2.5-7B prefill engine, 4 prompts x 2048 tokens:
    per layer, the KV write of every prompt token (reshape_and_cache_flash
    with the prompt's slot mapping) and causal varlen attention
    (flash_attn_varlen_func), GQA 28/4, D 128, bf16.  q/k/v are views of one
    fused [tokens, (28 + 8) * 128] projection output per layer, 28 layers of
    distinct inputs, so the append reads HBM, not cache.  Causal FLOPs:
    2 * Hq * D * n * (n + 1) per sequence (QK and PV)."""
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd.workloads import QWEN25_7B, split_tables
    dev = torch.device("cuda", 0)
    g = QWEN25_7B
    L, Hq, Hkv, D = g.n_layers, g.n_q_heads, g.n_kv_heads, g.head_dim
    lens = PREFILL_LENS
    T = sum(lens)
    rng = np.random.default_rng(args.seed)
    need = [-(-n // g.block_size) for n in lens]
    pool = 2 * sum(need)
    tables = split_tables(rng.permutation(pool)[:sum(need)], need)
    bs = g.block_size
    # every prompt position p: table[p // 16] * 16 + p % 16 (worker.py:628-633)
    slots = torch.from_numpy(np.concatenate(
        [np.asarray(t, dtype=np.int64)[np.arange(n) // bs] * bs + np.arange(n) % bs
         for t, n in zip(tables, lens)])).to(dev)
    cache = torch.empty((pool, *g.block_shape), dtype=torch.bfloat16, device=dev)
    view = cache.permute(1, 2, 0, 3, 4, 5)
    gen = torch.Generator(device=dev).manual_seed(args.seed + 2)
    qkv = torch.randn((L, T, (Hq + 2 * Hkv) * D), generator=gen, device=dev).to(torch.bfloat16)
    q = qkv[..., :Hq * D].view(L, T, Hq, D)
    k = qkv[..., Hq * D:(Hq + Hkv) * D].view(L, T, Hkv, D)
    v = qkv[..., (Hq + Hkv) * D:].view(L, T, Hkv, D)
    out = torch.empty((T, Hq, D), dtype=torch.bfloat16, device=dev)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    scale = 1.0 / math.sqrt(D)

    def append(i):
        layer = i % L
        A.reshape_and_cache_flash(k[layer], v[layer], view[layer, 0], view[layer, 1], slots)

    def attend(i):
        layer = i % L
        A.flash_attn_varlen_func(q[layer], k[layer], v[layer], cu, cu, max(lens), max(lens),
                                 softmax_scale=scale, causal=True, out=out)

    for i in range(L):
        append(i)
        attend(i)
    torch.cuda.synchronize()
    app_ms, _ = timer.run(append, 4 * L)
    att_ms, _ = timer.run(attend, 2 * L)
    flops = sum(2 * Hq * D * n * (n + 1) for n in lens)
    app_bytes = 2 * T * 2 * Hkv * D * 2 + 8 * T
    del cache, qkv, q, k, v, out
    torch.cuda.empty_cache()

    # one long prompt (the kernel's steady state): 8192 tokens, 8 layers of
    # distinct fused QKV views (600 MB, beyond the last-level cache)
    n8, L8 = PREFILL_LONG, 8
    qkv8 = torch.randn((L8, n8, (Hq + 2 * Hkv) * D), generator=gen, device=dev).to(torch.bfloat16)
    q8 = qkv8[..., :Hq * D].view(L8, n8, Hq, D)
    k8 = qkv8[..., Hq * D:(Hq + Hkv) * D].view(L8, n8, Hkv, D)
    v8 = qkv8[..., (Hq + Hkv) * D:].view(L8, n8, Hkv, D)
    out8 = torch.empty((n8, Hq, D), dtype=torch.bfloat16, device=dev)
    cu8 = torch.tensor([0, n8], dtype=torch.int32, device=dev)

    def attend_long(i):
        layer = i % L8
        A.flash_attn_varlen_func(q8[layer], k8[layer], v8[layer], cu8, cu8, n8, n8,
                                 softmax_scale=scale, causal=True, out=out8)

    attend_long(0)
    torch.cuda.synchronize()
    long_ms, _ = timer.run(attend_long, 2 * L8)
    del qkv8, q8, k8, v8, out8
    torch.cuda.empty_cache()

    # a ragged batch of 8 prompts (77 to 2048 tokens), 8 layers of distinct views
    rl = PREFILL_RAGGED
    Tr = sum(rl)
    qkvr = torch.randn((L8, Tr, (Hq + 2 * Hkv) * D), generator=gen, device=dev).to(torch.bfloat16)
    qr = qkvr[..., :Hq * D].view(L8, Tr, Hq, D)
    kr = qkvr[..., Hq * D:(Hq + Hkv) * D].view(L8, Tr, Hkv, D)
    vr = qkvr[..., (Hq + Hkv) * D:].view(L8, Tr, Hkv, D)
    outr = torch.empty((Tr, Hq, D), dtype=torch.bfloat16, device=dev)
    cur = torch.tensor(np.concatenate([[0], np.cumsum(rl)]), dtype=torch.int32, device=dev)

    def attend_ragged(i):
        layer = i % L8
        A.flash_attn_varlen_func(qr[layer], kr[layer], vr[layer], cur, cur, max(rl), max(rl),
                                 softmax_scale=scale, causal=True, out=outr)

    attend_ragged(0)
    torch.cuda.synchronize()
    ragged_ms, _ = timer.run(attend_ragged, 4 * L8)
    del qkvr, qr, kr, vr, outr
    torch.cuda.empty_cache()
    return {"append_ms": app_ms, "append_bytes": app_bytes, "attn_ms": att_ms, "flops": flops,
            "long_ms": long_ms, "long_flops": 2 * Hq * D * n8 * (n8 + 1),
            "ragged_ms": ragged_ms, "ragged_flops": sum(2 * Hq * D * n * (n + 1) for n in rl)}


# ------------------------------------------------------------------- block manager
BM_POOL_BLOCKS = 200_000           # 175 GiB of 0.875 MiB Qwen2.5-7B blocks on one GPU
BM_CPU_SLABS, BM_SLAB_BYTES = 128, 1 << 30   # aegaeon/aegaeon/config.py:37-39


def bench_block_manager(args, timer):
    """Host bookkeeping of one Qwen2.5-7B engine: a 200k-block GPU pool, the
    reference's CPU pool of 128 x 1 GiB slabs, 256 running requests
    (lognormal context mean 600).  A decode step grows every request by one
    token and calls allocate_blocks_batched on the batch
    (stage_engine.py:590); a turn moves the batch out to the CPU and back in
    (decode_scheduler.py:154,225).  Native manager vs the oracle's
    restatement of the reference's algorithm, same sequence, same ids."""
    from aegaeon_amd.block_manager import BLOCK_LOCATION_CPU, BlockManager
    from aegaeon_amd.workloads import QWEN25_7B, lognormal_lengths
    from oracle.block_manager_oracle import BlockManagerOracle
    shape = QWEN25_7B.block_shape
    rng = np.random.default_rng(args.seed)
    ctx = lognormal_lengths(rng, 256, 600.0, 1.0, 16, 4096)
    rids = list(range(256))
    n_steps, n_turns = 48, 3

    def needed(step):
        return [(int(c) + step + 1 + 15) // 16 for c in ctx]

    def run(make, alloc, move, steps, turns):
        m = make()
        m.register_gpu_space(0, BM_POOL_BLOCKS, shape)
        alloc(m, needed(0))
        t0 = time.perf_counter()
        for s in range(1, steps + 1):
            alloc(m, needed(s))
        t_step = (time.perf_counter() - t0) / steps
        t0 = time.perf_counter()
        for _ in range(turns):
            move(m, BLOCK_LOCATION_CPU)
            move(m, 0)
        t_turn = (time.perf_counter() - t0) / turns
        return m, t_step, t_turn

    nat, ns, nt = run(lambda: BlockManager(BM_CPU_SLABS, BM_SLAB_BYTES),
                      lambda m, need: m.allocate_blocks_by_count(rids, need, 0),
                      lambda m, loc: m.move_request_ids(rids, loc), n_steps, n_turns)
    ref, rs, rt = run(lambda: BlockManagerOracle(BM_CPU_SLABS, BM_SLAB_BYTES),
                      lambda m, need: m.allocate_blocks_batched(list(zip(rids, need)), 0),
                      lambda m, loc: m.move_requests(rids, loc), n_steps, n_turns)
    same = all(nat.get_block_table(r).blocks == ref.block_tables[r].blocks for r in rids)
    return {"native_us_per_step": ns * 1e6, "reference_us_per_step": rs * 1e6,
            "native_ms_per_turn": nt * 1e3, "reference_ms_per_turn": rt * 1e3,
            "blocks_per_turn": 2 * sum(len(ref.block_tables[r].blocks) for r in rids),
            "same_ids": same}


# ------------------------------------------------------------------ copy calibration
CALIB_BLOCKS, CALIB_BLOCK_BYTES = 256, 1 << 20


def bench_calib(args, timer):
    """A plain copy of known size for scaling the HBM byte counters: pack
    blocks 0..255 of 1 MiB (contiguous) into a staging buffer, i.e. read
    256 MiB and write 256 MiB with the block-copy kernel."""
    import torch
    from aegaeon_amd import ops
    dev = torch.device("cuda", 0)
    pool = torch.ones((4 * CALIB_BLOCKS, CALIB_BLOCK_BYTES), dtype=torch.uint8, device=dev)
    out = torch.empty((CALIB_BLOCKS, CALIB_BLOCK_BYTES), dtype=torch.uint8, device=dev)
    ids = np.arange(CALIB_BLOCKS, dtype=np.int64)

    def copy(i):
        ops.pack_blocks(pool, ids + CALIB_BLOCKS * (i % 4), out=out)

    copy(0)
    torch.cuda.synchronize()
    ms, _ = timer.run(copy, 8)
    del pool, out
    torch.cuda.empty_cache()
    return {"bytes": 2 * CALIB_BLOCKS * CALIB_BLOCK_BYTES, "ms": ms}


# ------------------------------------------------------------------- copy floor
FLOOR_BLOCKS, FLOOR_BLOCK_BYTES = 14, 1 << 20   # 14 MiB read + 14 MiB written = 29.36 MB


def bench_copy_floor(args, timer):
    """The copy floor at the headline append's bytes: the block-copy kernel
    copying 14 contiguous 1 MiB blocks (14,680,064 B read, the same written:
    29,360,128 B, the append's 29,362,176 B less its 2 KiB of slots) in its
    identity form (no id list, so no upload ahead of the kernel), with sources
    and destinations rotated over 32 regions (0.9 GB) as the append rotates
    its steps, so neither side is served from the last-level cache."""
    import torch
    from aegaeon_amd import ops
    dev = torch.device("cuda", 0)
    R = ROTATE_STEPS
    src = torch.ones((R, FLOOR_BLOCKS, FLOOR_BLOCK_BYTES), dtype=torch.uint8, device=dev)
    outs = torch.empty((R, FLOOR_BLOCKS, FLOOR_BLOCK_BYTES), dtype=torch.uint8, device=dev)

    def copy(i):
        r = i % R
        ops.copy_blocks(src[r], outs[r], None, None)

    def vendor(i):  # hipMemcpyAsync device to device (torch copy_ of contiguous tensors)
        r = i % R
        outs[r].copy_(src[r])

    for i in range(R):
        copy(i)
        vendor(i)
    torch.cuda.synchronize()
    ms, _ = timer.run(copy, args.steps)
    vendor_ms, _ = timer.run(vendor, args.steps)
    outs.zero_()
    for i in range(R):
        copy(i)
    torch.cuda.synchronize()
    if not torch.equal(outs, src):
        raise RuntimeError("copy floor: the copy is wrong")
    del src, outs
    torch.cuda.empty_cache()
    # the launch floor: the same kernel moving one 16-byte block (one
    # workgroup) back to back
    tiny = torch.ones((1, 16), dtype=torch.uint8, device=dev)
    tiny_out = torch.empty_like(tiny)
    ops.copy_blocks(tiny, tiny_out, None, None)
    torch.cuda.synchronize()
    floor_ms, _ = timer.run(lambda i: ops.copy_blocks(tiny, tiny_out, None, None), args.steps)
    del tiny, tiny_out
    return {"bytes": 2 * FLOOR_BLOCKS * FLOOR_BLOCK_BYTES, "ms": ms, "vendor_ms": vendor_ms,
            "launch_floor_ms": floor_ms}


# ---------------------------------------------------------------------- CPU baseline
def _median_time(fn, warmup=3, runs=10, min_s=1.0):
    """3 warm-ups, then the median of at least ``runs`` timed calls (more
    while under ``min_s`` seconds in total)."""
    for _ in range(warmup):
        fn()
    ts = []
    t_end = time.perf_counter() + min_s
    while len(ts) < runs or (time.perf_counter() < t_end and len(ts) < 1000):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return float(np.median(ts)), len(ts)


def cpu_baseline(args):
    """The reference's path restated with torch on the host CPU (the oracle's
    torch_cpu module), timed in this process on every core of the affinity
    mask: 3 warm-ups, then the median of at least 10 runs.  The headline
    figure is the Qwen2.5-7B all-layer append into the full 19,014-block pool
    (17.4 GB of host memory); ``ops`` holds one layer of the Qwen2.5-7B decode
    attention (float32 from bf16, 128 sequences) and the Llama-2-13B swap as
    host memcpy of 12.5 MiB blocks (a 64-block sample, as GB/s)."""
    import torch
    from aegaeon_amd.workloads import llama_swap_workload, qwen_append_batch, \
        qwen_attention_batch, successive_step_slots
    from oracle import torch_cpu as tc
    cores = len(os.sched_getaffinity(0))
    prev = torch.get_num_threads()
    torch.set_num_threads(cores)
    try:
        gen = torch.Generator().manual_seed(args.seed)
        wb = qwen_append_batch(args.seed)
        g = wb.geometry
        R = ROTATE_STEPS
        storage = torch.empty((wb.n_pool_blocks, *g.block_shape), dtype=torch.bfloat16)
        keys = torch.randn((R, g.n_layers, wb.batch, g.n_kv_heads, g.head_dim),
                           generator=gen).to(torch.bfloat16)
        vals = torch.randn(keys.shape, generator=gen).to(torch.bfloat16)
        slots = torch.from_numpy(successive_step_slots(wb, R))
        step = [0]

        def app():
            r = step[0] % R
            step[0] += 1
            tc.append_layers(keys[r], vals[r], storage, slots[r])

        t_app, n_app = _median_time(app)
        del storage, keys, vals
        ab = qwen_attention_batch(args.seed)
        ag = ab.geometry
        kc = torch.randn((ab.n_pool_blocks, 16, ag.n_kv_heads, ag.head_dim),
                         generator=gen).to(torch.bfloat16)
        vc = torch.randn(kc.shape, generator=gen).to(torch.bfloat16)
        q = torch.randn((ab.batch, ag.n_q_heads, ag.head_dim), generator=gen).to(torch.bfloat16)
        bt = torch.from_numpy(ab.padded_tables())
        sl = torch.from_numpy(ab.seq_lens)
        scale = 1.0 / math.sqrt(ag.head_dim)
        t_att, n_att = _median_time(lambda: tc.paged_decode_attention(q, kc, vc, bt, sl, scale))
        del kc, vc
        wl = llama_swap_workload(args.seed)
        bb = wl.geometry.block_bytes
        n_s = 64
        src_pool = torch.ones((2 * n_s, bb), dtype=torch.uint8)
        dst_pool = torch.zeros((n_s, bb), dtype=torch.uint8)
        src_ids = np.random.default_rng(args.seed).permutation(2 * n_s)[:n_s]
        t_swp, n_swp = _median_time(lambda: tc.swap_blocks(src_ids, range(n_s), src_pool,
                                                           dst_pool))
        del src_pool, dst_pool
    finally:
        torch.set_num_threads(prev)
    return {"value": round(wb.append_bytes() / t_app / 1e9, 3), "unit": "GB/s",
            "cores": cores, "kind": "port",
            "sample": f"torch CPU restatement of the append (oracle/torch_cpu.py) on {cores} "
                      f"threads: the full 256-token x 28-layer Qwen2.5-7B append into the "
                      f"{wb.n_pool_blocks}-block pool, {R} successive decode steps rotated as "
                      f"on the GPU, median of {n_app} runs after 3 warm-ups "
                      f"({t_app * 1e3:.2f} ms per step)",
            "cpu_model": _cpu_model(),
            "ops": {
                "paged_decode_attention_fp32": {
                    "workload": "one layer of the Qwen2.5-7B decode batch (128 seqs, "
                                "sum len 189059), float32 from bf16",
                    "us_per_layer": round(t_att * 1e6, 1),
                    "GB/s": round(ab.attention_bytes() / t_att / 1e9, 3), "runs": n_att},
                "swap_host_memcpy": {
                    "workload": f"Llama-2-13B swap restated as host-to-host block copies, "
                                f"{n_s} of the 4096 12.5 MiB blocks",
                    "ms": round(t_swp * 1e3, 2),
                    "GB/s": round(n_s * bb / t_swp / 1e9, 2), "runs": n_swp}}}


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _traffic():
    """HBM bytes per append launch from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or None."""
    p = ROOT / "profiles" / "kv_append_qwen_pmc.txt"
    if not p.exists():
        return None
    for line in p.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--nwg", type=int, default=0,
                   help="attention workgroups (0 = one per CU)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--swap-seqs", type=int, default=32)
    p.add_argument("--swap-blocks", type=int, default=-1,
                   help="blocks of the Llama-2-13B swap sent through pinned host memory "
                        "(-1 = all 4096 when the host can pin them; 0 = skip)")
    p.add_argument("--only", default="all",
                   help="comma list of append,attention,pack,defrag,gather,overlap,prefill,"
                        "prepare,bm,calib,floor or 'all'")
    args = p.parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "aegaeon_amd's KV data path is per-GPU and runs no "
                                   "collectives: the benchmark measures one GPU, so --gpus must "
                                   "be 1"}), flush=True)
        return 2
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}), flush=True)
        return 2
    from aegaeon_amd import _lib
    _lib.load()
    torch.cuda.set_device(0)
    log(f"device: {torch.cuda.get_device_name(0)}")
    only = set(args.only.split(",")) if args.only != "all" else \
        {"append", "attention", "pack", "defrag", "gather", "overlap", "prefill", "prepare", "bm",
         "calib", "floor"}
    timer = Timer()
    log(f"spin calibration: {timer.cycles_per_ms:.0f} cycles/ms")
    res = {}
    for name, fn in (("append", bench_append), ("attention", bench_attention),
                     ("gather", bench_gather), ("pack", bench_pack), ("defrag", bench_defrag),
                     ("overlap", bench_overlap), ("prefill", bench_prefill),
                     ("prepare", bench_prepare),
                     ("bm", bench_block_manager),
                     ("calib", bench_calib), ("floor", bench_copy_floor)):
        if name in only:
            t0 = time.perf_counter()
            res[name] = fn(args, timer)
            log(f"{name} done in {time.perf_counter() - t0:.1f} s")
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args)
        log(f"cpu baseline done: {cpu['value']} GB/s")

    line = {"metric": METRIC, "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "higher_is_better": True, "scaling": "weak",
            "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic: seeded N(0,1) K/V and queries, seeded lognormal lengths and "
                    "random-permutation block tables"}
    ops_out = {}
    if "append" in res:
        a = res["append"]
        value = a["bytes"] / (a["ms"] * 1e-3) / 1e9
        line.update({
            "value": round(value, 1), "ms_per_step": round(a["ms"], 6),
            "config": {"workload": "Qwen2.5-7B-shaped decode-step KV append, all 28 layers in "
                                   "one launch, 256 sequences (lognormal mean 600), bf16",
                       "layers": 28, "kv_heads": 4, "head_dim": 128, "block_size": 16,
                       "batch": a["wb"].batch, "pool_blocks": a["wb"].n_pool_blocks,
                       "bytes_per_step": a["bytes"], "rotated_steps": ROTATE_STEPS},
            "roofline": {"bound": "hbm", "achieved": round(value, 1), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(value / HBM_PEAK_GBS, 4),
                         "traffic": _traffic()},
        })
        ops_out["append_kernel_us"] = round(a["ms"] * 1e3, 2)
        ops_out["append_same_inputs_every_step_us"] = round(a["hot_ms"] * 1e3, 2)
        ops_out["append_per_layer_28_launches_us"] = round(a["per_layer_step_ms"] * 1e3, 2)
    if "attention" in res:
        t = res["attention"]
        gbs = t["bytes_per_layer"] / (t["us_per_layer"] * 1e-6) / 1e9
        ops_out["paged_decode_attention"] = {
            "workload": "Qwen2.5-7B GQA 28/4, D 128, bf16, 128 seqs, lognormal mean 1500 "
                        "(sum len 189059), 28 layers back to back, one decode plan per step "
                        "(its build included)",
            "us_per_layer": round(t["us_per_layer"], 2),
            "bytes_per_layer": t["bytes_per_layer"], "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "unplanned_us_per_layer": round(t["unplanned_us_per_layer"], 2),
            "flash_attn_with_kvcache_us_per_layer": round(t["kvcache_us"], 2)}
        ops_out["decode_layer_append_then_attention"] = {
            "workload": "the same batch, each layer's new token appended then attended over "
                        "seq_len tokens, one decode plan per step",
            "two_launches_us_per_layer": round(t["two_launch_us"], 2),
            "fused_us_per_layer": round(t["fused_us"], 2),
            "bit_identical": True}
        if "value" not in line:
            line.update({"value": round(t["us_per_layer"], 2), "unit": "us/layer",
                         "higher_is_better": False})
    if "gather" in res:
        gt = res["gather"]
        gbs = gt["bytes"] / (gt["ms"] * 1e-3) / 1e9
        ops_out["gather_tokens_one_layer"] = {
            "workload": "Qwen2.5-7B append batch, 256 seqs, one layer K+V",
            "us": round(gt["ms"] * 1e3, 2), "bytes": gt["bytes"], "GB/s": round(gbs, 1),
            "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "torch_index_select_whole_blocks_us": round(gt["torch_ms"] * 1e3, 2),
            "torch_index_select_GB/s": round(gt["torch_bytes"] / (gt["torch_ms"] * 1e-3) / 1e9, 1),
            "contiguous_copy_same_bytes_us": round(gt["contig_ms"] * 1e3, 2),
            "contiguous_copy_same_bytes_GB/s": round(
                gt["contig_bytes"] / (gt["contig_ms"] * 1e-3) / 1e9, 1)}
    if "pack" in res:
        pk = res["pack"]
        pg = pk["bytes"] / (pk["pack_ms"] * 1e-3) / 1e9
        sg = pk["bytes"] / (pk["scatter_ms"] * 1e-3) / 1e9
        ops_out["swap_pack_scatter"] = {
            "workload": f"Llama-2-13B, {pk['wl'].n_blocks} blocks x 12.5 MiB fp16",
            "pack_ms": round(pk["pack_ms"], 3), "scatter_ms": round(pk["scatter_ms"], 3),
            "bytes": pk["bytes"], "pack_GB/s": round(pg, 1), "scatter_GB/s": round(sg, 1),
            "pack_frac_hbm": round(pg / HBM_PEAK_GBS, 4),
            "scatter_frac_hbm": round(sg / HBM_PEAK_GBS, 4),
            "torch_index_select_ms": round(pk["torch_pack_ms"], 3),
            "torch_index_select_GB/s": round(pk["bytes"] / (pk["torch_pack_ms"] * 1e-3) / 1e9, 1),
            "torch_index_copy_ms": round(pk["torch_scatter_ms"], 3),
            "torch_index_copy_GB/s": round(pk["bytes"] / (pk["torch_scatter_ms"] * 1e-3) / 1e9, 1),
            "contiguous_copy_same_bytes_ms": round(pk["contig_ms"], 3),
            "contiguous_copy_same_bytes_GB/s": round(
                pk["contig_bytes"] / (pk["contig_ms"] * 1e-3) / 1e9, 1),
        }
        sw = pk["swap"]
        if sw is not None:
            n, bb = sw["blocks"], pk["wl"].geometry.block_bytes
            rate = lambda ms: round(n * bb / (ms * 1e-3) / 1e9, 2)  # noqa: E731
            ops_out["swap_through_pinned_host"] = {
                "workload": f"Llama-2-13B swap through ops.swap: {n} of the {sw['of_blocks']} "
                            f"scattered 12.5 MiB blocks out to pinned host and back into a "
                            f"disjoint free set (scale {n / sw['of_blocks']:g})",
                "blocks": n, "bytes_each_way": n * bb,
                "swap_out_ms": round(sw["swap_out_ms"], 2), "swap_out_GB/s": rate(sw["swap_out_ms"]),
                "swap_in_ms": round(sw["swap_in_ms"], 2), "swap_in_GB/s": rate(sw["swap_in_ms"]),
                "legs": {"pack_ms": round(sw["pack_ms"], 3),
                         "dma_d2h_ms": round(sw["dma_d2h_ms"], 2),
                         "dma_d2h_GB/s": rate(sw["dma_d2h_ms"]),
                         "dma_h2d_ms": round(sw["dma_h2d_ms"], 2),
                         "dma_h2d_GB/s": rate(sw["dma_h2d_ms"]),
                         "scatter_ms": round(sw["scatter_ms"], 3)},
                "frac_pcie5_x16": round(rate(sw["swap_out_ms"]) / PCIE_PEAK_GBS, 4),
                "pin_seconds": round(sw["pin_s"], 1)}
            fl = sw.get("file")
            if fl:
                nf = fl["blocks"]
                frate = lambda ms: round(nf * bb / (ms * 1e-3) / 1e9, 2)  # noqa: E731
                ops_out["swap_through_shm_file"] = {
                    "workload": f"the same swap for {nf} blocks into a /dev/shm file mapping "
                                f"(the reference's shared swap space) through a 256 MiB pinned "
                                f"bounce buffer",
                    "swap_out_ms": round(fl["swap_out_ms"], 2),
                    "swap_out_GB/s": frate(fl["swap_out_ms"]),
                    "swap_in_ms": round(fl["swap_in_ms"], 2),
                    "swap_in_GB/s": frate(fl["swap_in_ms"])}
    if "defrag" in res:
        d = res["defrag"]
        dg = d["defrag_bytes"] / (d["defrag_ms"] * 1e-3) / 1e9
        ag = d["yi_append_bytes"] / (d["yi_append_ms"] * 1e-3) / 1e9
        tg = d["yi_attn_bytes"] / (d["yi_attn_us_per_layer"] * 1e-6) / 1e9
        ops_out["unified_pool_defrag"] = {
            "workload": "Yi-1.5-9B + Qwen2.5-7B + Llama-2-13B blocks in 1 GiB slabs, 50% live",
            "moved_blocks": d["moved_blocks"], "ms": round(d["defrag_ms"], 3),
            "bytes": d["defrag_bytes"], "GB/s": round(dg, 1), "frac_hbm": round(dg / HBM_PEAK_GBS, 4),
            "torch_index_select_index_copy_ms": round(d["torch_defrag_ms"], 3),
            "torch_GB/s": round(d["defrag_bytes"] / (d["torch_defrag_ms"] * 1e-3) / 1e9, 1),
            "yi_append_us": round(d["yi_append_ms"] * 1e3, 2), "yi_append_GB/s": round(ag, 1),
            "yi_attention_us_per_layer": round(d["yi_attn_us_per_layer"], 2),
            "yi_attention_GB/s": round(tg, 1), "yi_attention_frac_hbm": round(tg / HBM_PEAK_GBS, 4)}
    if "prepare" in res:
        ops_out["prepare_inputs_us_per_step"] = {
            k: {"device_from_request_lists": round(v["device"], 1),
                "device_from_arrays": round(v["device_from_arrays"], 1),
                "reference_host_loops": round(v["reference_host"], 1)}
            for k, v in res["prepare"].items()}
    if "overlap" in res:
        ov = res["overlap"]
        hidden = (ov["attn_ms"] + ov["swap_ms"] - ov["both_ms"]) / min(ov["attn_ms"], ov["swap_ms"])
        ops_out["swap_overlapped_with_attention"] = {
            "workload": "28 layers of Qwen2.5-7B decode attention (128 seqs) on the compute "
                        "stream; 128 scattered Qwen2.5-7B blocks (112 MiB) swapped out to "
                        "pinned host on a side stream",
            "attention_alone_ms": round(ov["attn_ms"], 3), "swap_alone_ms": round(ov["swap_ms"], 3),
            "together_ms": round(ov["both_ms"], 3),
            "swap_GB/s_alone": round(ov["swap_bytes"] / (ov["swap_ms"] * 1e-3) / 1e9, 1),
            "fraction_of_shorter_hidden": round(hidden, 3)}
    if "prefill" in res:
        pf = res["prefill"]
        tf = pf["flops"] / (pf["attn_ms"] * 1e-3) / 1e12
        ag = pf["append_bytes"] / (pf["append_ms"] * 1e-3) / 1e9
        ops_out["prefill_qwen_4x2048"] = {
            "workload": "Qwen2.5-7B prompt run, 4 prompts x 2048 tokens (profiled shape i2048b4), "
                        "GQA 28/4, D 128, bf16, 28 layers of distinct q/k/v views of a fused QKV",
            "attention_us_per_layer": round(pf["attn_ms"] * 1e3, 2),
            "attention_flops_per_layer": pf["flops"], "TFLOP/s": round(tf, 1),
            "frac_mfma_bf16": round(tf / MFMA_BF16_PEAK_TFLOPS, 4),
            "kv_write_us_per_layer": round(pf["append_ms"] * 1e3, 2),
            "kv_write_bytes_per_layer": pf["append_bytes"], "kv_write_GB/s": round(ag, 1),
            "kv_write_frac_hbm": round(ag / HBM_PEAK_GBS, 4)}
        tl = pf["long_flops"] / (pf["long_ms"] * 1e-3) / 1e12
        ops_out["prefill_qwen_1x8192"] = {
            "workload": "Qwen2.5-7B prompt run, one 8192-token prompt (the attention kernel's "
                        "steady state), GQA 28/4, D 128, bf16, causal, 8 layers of distinct q/k/v "
                        "views of a fused QKV",
            "attention_us_per_layer": round(pf["long_ms"] * 1e3, 2),
            "attention_flops_per_layer": pf["long_flops"], "TFLOP/s": round(tl, 1),
            "frac_mfma_bf16": round(tl / MFMA_BF16_PEAK_TFLOPS, 4)}
        tr = pf["ragged_flops"] / (pf["ragged_ms"] * 1e-3) / 1e12
        ops_out["prefill_qwen_ragged8"] = {
            "workload": "Qwen2.5-7B prompt run, 8 prompts of %s tokens, GQA 28/4, D 128, bf16, "
                        "causal, 8 layers of distinct q/k/v views of a fused QKV"
                        % "/".join(str(n) for n in PREFILL_RAGGED),
            "attention_us_per_layer": round(pf["ragged_ms"] * 1e3, 2),
            "attention_flops_per_layer": pf["ragged_flops"], "TFLOP/s": round(tr, 1),
            "frac_mfma_bf16": round(tr / MFMA_BF16_PEAK_TFLOPS, 4)}
    if "bm" in res:
        b = res["bm"]
        ops_out["block_manager"] = {
            "workload": "Qwen2.5-7B engine, 200k-block GPU pool, 128 x 1 GiB CPU slabs, 256 "
                        "requests; step = allocate_blocks_batched after one token each, turn = "
                        "batch moved out to CPU and back in",
            "native_us_per_step": round(b["native_us_per_step"], 1),
            "reference_algorithm_us_per_step": round(b["reference_us_per_step"], 1),
            "native_ms_per_turn": round(b["native_ms_per_turn"], 3),
            "reference_algorithm_ms_per_turn": round(b["reference_ms_per_turn"], 3),
            "blocks_moved_per_turn": b["blocks_per_turn"], "same_block_ids": b["same_ids"]}
    if "calib" in res:
        c = res["calib"]
        cg = c["bytes"] / (c["ms"] * 1e-3) / 1e9
        ops_out["copy_calibration"] = {
            "workload": "pack of 256 contiguous 1 MiB blocks (256 MiB read + 256 MiB write)",
            "us": round(c["ms"] * 1e3, 2), "bytes": c["bytes"], "GB/s": round(cg, 1),
            "frac_hbm": round(cg / HBM_PEAK_GBS, 4)}
    if "floor" in res:
        f = res["floor"]
        fg = f["bytes"] / (f["ms"] * 1e-3) / 1e9
        ops_out["copy_floor_at_append_bytes"] = {
            "workload": "the library's contiguous copy (copy_blocks without id lists: 1 KiB "
                        "per one-wave workgroup), 14 contiguous 1 MiB blocks (29,360,128 B moved, the "
                        "headline append's bytes less its slots), 32 rotated regions",
            "us": round(f["ms"] * 1e3, 2), "bytes": f["bytes"], "GB/s": round(fg, 1),
            "frac_hbm": round(fg / HBM_PEAK_GBS, 4)}
        vg = f["bytes"] / (f["vendor_ms"] * 1e-3) / 1e9
        ops_out["vendor_copy_floor_at_append_bytes"] = {
            "workload": "hipMemcpyAsync device to device (torch copy_) of the same 29,360,128 B, "
                        "32 rotated regions",
            "us": round(f["vendor_ms"] * 1e3, 2), "GB/s": round(vg, 1),
            "frac_hbm": round(vg / HBM_PEAK_GBS, 4)}
        ops_out["launch_floor_us"] = {
            "workload": "the block-copy kernel moving one 16-byte block (one workgroup) back to "
                        "back: the fixed cost of a launch that moves no data",
            "one_workgroup": round(f["launch_floor_ms"] * 1e3, 2)}
    line["ops"] = ops_out
    if cpu is not None:
        line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
