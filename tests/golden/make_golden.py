"""Write the golden fixture for the 1-layer / 2-head / D=64 fp16 plumbing case.

The reference holds no golden vectors for this path, so the expected outputs
here are computed by deliberately naive scalar loops over FLAT indices of the
reference's storage layout ``[N, L, 2, 16, Hkv, D]`` (aegaeon/aegaeon/
worker.py:389-395) — an independent statement of the layout, not the oracle's
vectorised reshape/transpose code:

  flat(blk, l, kv, off, h, d) = ((((blk*L + l)*2 + kv)*16 + off)*Hkv + h)*D + d

  * slot mapping: slot = bt[pos // 16] * 16 + pos % 16 (worker.py:628-633);
  * append: element (t, h, d) of the new key lands at flat(slot//16, 0, 0,
    slot%16, h, d) (vLLM reshape_and_cache_flash semantics);
  * gather: token p of sequence b is read from flat(bt[p//16], 0, kv, p%16, h, d);
  * swap-out: byte j of block src[i] goes to byte j of host block dst[i]
    (aegaeon/ops/swap.cu:36-58), done one uint16 at a time.

Run: ``python tests/golden/make_golden.py`` (writes tests/golden/cfg1_tiny.npz).
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))

from aegaeon_amd.workloads import tiny_batch  # noqa: E402

OUT = HERE / "cfg1_tiny.npz"


def main() -> None:
    wb = tiny_batch(0)
    g = wb.geometry
    L, H, D, BS = g.n_layers, g.n_kv_heads, g.head_dim, g.block_size
    N = wb.n_pool_blocks
    rng = np.random.default_rng(1000)
    pool = rng.standard_normal(N * g.block_elems).astype(np.float16).view(np.uint16)
    new_k = rng.standard_normal((wb.batch, H, D)).astype(np.float16).view(np.uint16)
    new_v = rng.standard_normal((wb.batch, H, D)).astype(np.float16).view(np.uint16)

    def flat(blk, l, kv, off, h, d):
        return ((((blk * L + l) * 2 + kv) * BS + off) * H + h) * D + d

    # slot mapping, one token per sequence at position context_len
    slots = []
    for bt, pos in zip(wb.block_tables, wb.context_lens):
        pos = int(pos)
        slots.append(bt[pos // BS] * BS + pos % BS)
    slots = np.asarray(slots, dtype=np.int64)

    # append
    after = pool.copy()
    written = []
    for t, s in enumerate(slots):
        for h in range(H):
            for d in range(D):
                ik, iv = flat(s // BS, 0, 0, s % BS, h, d), flat(s // BS, 0, 1, s % BS, h, d)
                after[ik] = new_k[t, h, d]
                after[iv] = new_v[t, h, d]
                written += [ik, iv]
    written = np.asarray(sorted(written), dtype=np.int64)

    # gather every sequence's tokens (context + the appended one)
    seq_lens = wb.context_lens + 1
    total = int(seq_lens.sum())
    out_k = np.zeros((total, H, D), dtype=np.uint16)
    out_v = np.zeros((total, H, D), dtype=np.uint16)
    base = 0
    for b, ln in enumerate(seq_lens):
        bt = wb.block_tables[b]
        for p in range(int(ln)):
            for h in range(H):
                for d in range(D):
                    out_k[base + p, h, d] = after[flat(bt[p // BS], 0, 0, p % BS, h, d)]
                    out_v[base + p, h, d] = after[flat(bt[p // BS], 0, 1, p % BS, h, d)]
        base += int(ln)

    # swap-out of every used block to host blocks 0..n-1, element by element
    src = [x for bt in wb.block_tables for x in bt]
    dst = list(range(len(src)))
    be = g.block_elems
    host = np.zeros(len(dst) * be, dtype=np.uint16)
    for s, d in zip(src, dst):
        for j in range(be):
            host[d * be + j] = after[s * be + j]

    np.savez_compressed(
        OUT,
        pool=pool, new_k=new_k, new_v=new_v, slots=slots,
        append_idx=written, append_val=after[written],
        seq_lens=seq_lens, tables=wb.padded_tables(), out_k=out_k, out_v=out_v,
        swap_src=np.asarray(src, dtype=np.int64), swap_dst=np.asarray(dst, dtype=np.int64),
        host_after_swap=host,
        geometry=np.asarray([N, L, H, D, BS], dtype=np.int64),
        context_lens=wb.context_lens)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
