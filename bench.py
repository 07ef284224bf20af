"""Benchmark of the MI355X KV-cache data path (one GPU).

Headline (``value``): KV append throughput in GB/s for one decode step of the
Qwen2.5-7B-shaped batch (28 layers, 4 KV heads, D 128, bf16, 256 sequences,
context lengths lognormal mean 600, pool = 2x need), all layers in one launch.
A "step" is one such append.  Algorithmic bytes per step: read K and V, write
them into the paged pool, read the slot mapping:
``2 * B * L * 2 * Hkv * D * 2 + 8 * B``.

Secondary lines in the same JSON object (``ops``): paged decode attention
microseconds per layer for the Qwen2.5-7B attention batch (128 sequences,
lognormal mean 1500, up to 8192 tokens), block pack/scatter for the
Llama-2-13B swap workload, defrag of the unified multi-model pool.

Timing: W untimed warm-up steps, then K timed steps bracketed by
``torch.cuda.synchronize()``; kernel time per launch is taken with HIP events
recorded on the stream the kernels run on (torch's current stream).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import platform
import sys
import time

import numpy as np

HBM_PEAK_GBS = 8000.0


def _events_ms(fn, iters: int) -> float:
    import torch
    st = torch.cuda.current_stream()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(iters):
        fn()
    e1.record(st)
    e1.synchronize()
    return e0.elapsed_time(e1) / iters


def bench_append(args, device):
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd.workloads import qwen_append_batch
    wb = qwen_append_batch(args.seed)
    g = wb.geometry
    cache = torch.empty((wb.n_pool_blocks, *g.block_shape), dtype=torch.bfloat16, device=device)
    gen = torch.Generator(device=device).manual_seed(args.seed)
    key = torch.randn((g.n_layers, wb.batch, g.n_kv_heads, g.head_dim), generator=gen,
                      device=device).to(torch.bfloat16)
    val = torch.randn(key.shape, generator=gen, device=device).to(torch.bfloat16)
    slots = torch.from_numpy(wb.slot_mapping()).to(device)

    def step():
        A.append_kv(key, val, cache, slots)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    kernel_ms = _events_ms(step, args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    nbytes = wb.append_bytes()
    # per-layer launches (vLLM's call pattern) for comparison
    view = cache.permute(1, 2, 0, 3, 4, 5)

    def per_layer():
        for layer in range(g.n_layers):
            A.reshape_and_cache_flash(key[layer], val[layer], view[layer, 0], view[layer, 1], slots)

    per_layer()
    torch.cuda.synchronize()
    per_layer_ms = _events_ms(per_layer, max(1, args.steps // 4))
    del cache
    return {
        "wb": wb, "bytes": nbytes, "kernel_ms": kernel_ms, "wall_s": wall,
        "per_layer_launch_ms": per_layer_ms,
    }


def bench_attention(args, device):
    import torch
    from aegaeon_amd import attention as A
    from aegaeon_amd.workloads import qwen_attention_batch
    wb = qwen_attention_batch(args.seed)
    g = wb.geometry
    N = wb.n_pool_blocks
    cache = torch.empty((N, *g.block_shape), dtype=torch.bfloat16, device=device)
    gen = torch.Generator(device=device).manual_seed(args.seed + 1)
    # random K/V in the used blocks (all layers), in slices to bound the temporary
    for i in range(0, N, 1024):
        sl = cache[i:i + 1024]
        sl.copy_(torch.randn(sl.shape, generator=gen, device=device, dtype=torch.float32)
                 .to(torch.bfloat16))
    q = torch.randn((g.n_layers, wb.batch, g.n_q_heads, g.head_dim), generator=gen,
                    device=device).to(torch.bfloat16)
    bt = torch.from_numpy(wb.padded_tables()).to(device)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(device)
    max_len = int(wb.seq_lens.max())
    view = cache.permute(1, 2, 0, 3, 4, 5)
    scale = 1.0 / math.sqrt(g.head_dim)
    outs = torch.empty_like(q)
    ws = torch.empty(max(1, A.attention_workspace_bytes(wb.batch, g.n_q_heads, g.head_dim,
                                                        max_len, args.bps)),
                     dtype=torch.uint8, device=device)

    def all_layers():
        for layer in range(g.n_layers):
            A.paged_decode_attention(q[layer], view[layer, 0], view[layer, 1], bt, sl, scale,
                                     max_len, out=outs[layer], blocks_per_split=args.bps,
                                     workspace=ws)

    all_layers()
    torch.cuda.synchronize()
    ms = _events_ms(all_layers, max(1, args.steps // 4))
    per_layer_us = ms * 1e3 / g.n_layers
    nbytes = wb.attention_bytes()
    del cache
    return {"wb": wb, "bytes_per_layer": nbytes, "us_per_layer": per_layer_us}


def cpu_baseline_append(args):
    """The oracle's append (numpy, one thread) on a bounded sample: the same
    256 tokens x 28 layers, into a compact pool holding only the touched
    blocks; repeated for ~10 s."""
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import kv_oracle as ko
    from aegaeon_amd.workloads import qwen_append_batch
    wb = qwen_append_batch(args.seed)
    g = wb.geometry
    slots = wb.slot_mapping()
    blocks = np.unique(slots // 16)
    remap = {int(b): i for i, b in enumerate(blocks)}
    cslots = np.asarray([remap[int(s // 16)] * 16 + int(s % 16) for s in slots], dtype=np.int64)
    storage = np.zeros((len(blocks), *g.block_shape), dtype=np.uint16)
    rng = np.random.default_rng(args.seed)
    key = rng.integers(0, 1 << 16, size=(g.n_layers, wb.batch, g.n_kv_heads, g.head_dim),
                       dtype=np.uint16)
    val = key[::-1].copy()
    reps, t0 = 0, time.perf_counter()
    while True:
        ko.append_layers(key, val, storage, cslots)
        reps += 1
        el = time.perf_counter() - t0
        if el > args.cpu_seconds:
            break
    return {"value": wb.append_bytes() * reps / el / 1e9, "unit": "GB/s", "cores": 1,
            "kind": "port",
            "sample": f"oracle append_layers (numpy, 1 thread), {reps} reps of the full 256-token "
                      f"x 28-layer append into a compact {len(blocks)}-block pool, {el:.1f} s"}


def main(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--bps", type=int, default=0, help="attention blocks per split (0 = default)")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only", choices=["append", "attention", "all"], default="all")
    args = p.parse_args(argv)
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: the KV data path is per-GPU "
                                   "and runs no collectives; --gpus must be 1"}))
        return 2
    import torch
    if not torch.cuda.is_available():
        print(json.dumps({"error": "no GPU visible"}))
        return 2
    from aegaeon_amd import _lib
    _lib.load()
    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    print(f"# device: {torch.cuda.get_device_name(device)}", file=sys.stderr, flush=True)

    res = {}
    if args.only in ("append", "all"):
        res["append"] = bench_append(args, device)
        print(f"# append done: {res['append']['kernel_ms']*1e3:.2f} us/launch", file=sys.stderr,
              flush=True)
    if args.only in ("attention", "all"):
        res["attention"] = bench_attention(args, device)
        print(f"# attention done: {res['attention']['us_per_layer']:.2f} us/layer",
              file=sys.stderr, flush=True)
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_append(args)
        print(f"# cpu baseline done: {cpu['value']:.3f} GB/s", file=sys.stderr, flush=True)

    line = {"metric": "KV gather/append GB/s (%HBM peak); paged decode-attn us/layer @Qwen2.5-7B",
            "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
            "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
            "data": "synthetic (seeded N(0,1) K/V, seeded lognormal lengths and block tables)"}
    if "append" in res:
        a = res["append"]
        gbs = a["bytes"] / (a["kernel_ms"] * 1e-3) / 1e9
        line.update({
            "value": round(gbs, 2), "ms_per_step": round(a["kernel_ms"], 6),
            "config": {"workload": "Qwen2.5-7B decode-step KV append, all 28 layers in one launch",
                       "batch": a["wb"].batch, "layers": 28, "kv_heads": 4, "head_dim": 128,
                       "block_size": 16, "pool_blocks": a["wb"].n_pool_blocks,
                       "bytes_per_step": a["bytes"]},
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                         "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
        })
        line["ops"] = {"append_per_layer_launches_us": round(a["per_layer_launch_ms"] * 1e3, 2)}
    if "attention" in res:
        t = res["attention"]
        gbs = t["bytes_per_layer"] / (t["us_per_layer"] * 1e-6) / 1e9
        line.setdefault("ops", {})["paged_decode_attention"] = {
            "workload": "Qwen2.5-7B GQA 28/4, D 128, bf16, 128 seqs, lognormal mean 1500",
            "us_per_layer": round(t["us_per_layer"], 2), "bytes_per_layer": t["bytes_per_layer"],
            "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        if "value" not in line:
            line.update({"value": round(t["us_per_layer"], 2), "unit": "us/layer",
                         "higher_is_better": False})
    if cpu is not None:
        cpu["value"] = round(cpu["value"], 4)
        line["cpu_baseline"] = cpu
        line["cpu_baseline"]["cpu_model"] = platform.processor() or platform.machine()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
