"""Child process of tests/test_gpu_swap_file.py: a second worker on the same
node (here, the same GPU) that shares the swap-space file and the move events
of the parent, as two engines' workers share them in the reference
(aegaeon/aegaeon/worker.py:130-147,772-815, utils.py:306-331).

Protocol (one JSON object per line on stdin/stdout):
  child -> {"ready": true}                        after start-up
  parent -> {"handle": [device, pid, hex, word, serial], "file_ids": [...], "dev_ids": [...], "seed": s,
             "out_file_ids": [...], "out_seed": s2, "hold_cycles": c}
  child: swap-in of file_ids -> dev_ids waiting on the parent's event, check
         against the seeded bytes; then its own seeded blocks out to
         out_file_ids behind a held stream
  child -> {"ok": bool, "detail": str, "handle": [device, pid, hex, word, serial]}
  parent -> {"done": true}                        the child exits 0
"""
import json
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

SHAPE = (2, 2, 16, 4, 128)   # 64 KiB bf16 blocks
N_DEV = 64


def seeded_blocks(seed, n):
    import torch
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-2 ** 15, 2 ** 15, (n, *SHAPE), dtype=torch.int16, generator=g)


def send(obj):
    sys.stdout.write(json.dumps(obj) + "\n")
    sys.stdout.flush()


def main():
    import torch
    from aegaeon_amd import swap_pool
    from aegaeon_amd.worker_swap import KVSwapWorker
    path, n_slabs, slab = sys.argv[1], int(sys.argv[2]), int(sys.argv[3])
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    kv_swap = swap_pool.init_cpu_cache(n_slabs, slab, path)
    cache = torch.zeros((N_DEV, *SHAPE), dtype=torch.bfloat16, device=dev)
    worker = KVSwapWorker(cache, kv_swap, interprocess=True, bounce_bytes=1 << 20)
    torch.cuda.synchronize()
    send({"ready": True})

    msg = json.loads(sys.stdin.readline())
    d, pid, raw, word, serial = msg["handle"]
    handle = (int(d), int(pid), bytes.fromhex(raw), int(word), int(serial))
    ev_in = worker.swap_blocks([7], msg["file_ids"], msg["dev_ids"], [handle], True)
    ev_in.synchronize()
    worker.check_timeouts()
    opened = swap_pool.rebuild_event(handle)
    n_words = opened[0].n_words if opened else -1
    want = seeded_blocks(msg["seed"], len(msg["dev_ids"]))
    got = cache[torch.tensor(msg["dev_ids"], device=dev)].view(torch.int16).cpu()
    ok = bool(torch.equal(got, want)) and n_words == 2
    detail = "" if ok else f"{int((got != want).sum())} int16 words differ, array of {n_words} words"

    # this worker's own swap-out, held so that it is still pending when the
    # parent enqueues the swap-in that waits on it
    src_ids = list(range(32, 32 + len(msg["out_file_ids"])))
    cache[torch.tensor(src_ids, device=dev)] = \
        seeded_blocks(msg["out_seed"], len(src_ids)).to(dev).view(torch.bfloat16)
    torch.cuda.synchronize()
    with torch.cuda.stream(worker.swap_out_stream):
        torch.cuda._sleep(int(msg["hold_cycles"]))
    ev_out = worker.swap_blocks([8], src_ids, msg["out_file_ids"], [None], False)
    d2, pid2, raw2, w2, s2 = worker.export(ev_out)
    send({"ok": ok, "detail": detail, "handle": [d2, pid2, raw2.hex(), w2, s2]})
    sys.stdin.readline()                 # the parent is done with the event
    torch.cuda.synchronize()
    return 0


if __name__ == "__main__":
    sys.exit(main())
