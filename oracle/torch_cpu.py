"""The reference's path restated with torch on the host CPU — TEST
INFRASTRUCTURE ONLY (the timed CPU baseline of bench.py and a cross-check of
the numpy oracle in tests/test_oracle.py; the product never imports it).

The reference has no CPU implementation of this path: swap is
aegaeon/ops/swap.cu:25-59 and append/attention are vLLM CUDA kernels reached
from the forward (aegaeon/aegaeon/worker.py:517-523).  These functions are
the same semantics as torch CPU operators, vectorised so that a multi-threaded
torch build uses every host core:

* :func:`append_layers` — ``reshape_and_cache_flash`` for every layer of the
  ``[N, L, 2, 16, Hkv, D]`` storage (worker.py:389-395): one index_put per K
  and V over (layer, token), slot ``s`` at block ``s // 16`` offset ``s % 16``
  (worker.py:628-633), slots ``< 0`` skipped;
* :func:`paged_decode_attention` — ``flash_attn_with_kvcache`` for one query
  token per sequence, in float32 from the 16-bit cache (worker.py:410-418,
  694-711): per sequence, its blocks gathered through the block table, GQA
  query head ``h`` on kv head ``h // (Hq // Hkv)``;
* :func:`swap_blocks` — swap.cu's per-block copies as host-to-host block
  copies (``dst[dst_ids[i]] = src[src_ids[i]]``).

Pinned against the numpy oracle (kv_oracle) on seeded inputs: bit-exact for
the byte moves, and within float32 rounding for attention.
"""
from __future__ import annotations

import torch

BLOCK_SIZE = 16


def append_layers(key: torch.Tensor, value: torch.Tensor, storage: torch.Tensor,
                  slots: torch.Tensor) -> None:
    """key/value ``[L, T, Hkv, D]``; storage ``[N, L, 2, bs, Hkv, D]``;
    slots int64 ``[T]``."""
    L = key.size(0)
    bs = storage.size(3)
    keep = slots >= 0
    s = slots[keep]
    blk = (s // bs).view(1, -1)
    off = (s % bs).view(1, -1)
    layer = torch.arange(L).view(-1, 1)
    storage[blk, layer, 0, off] = key[:, keep]
    storage[blk, layer, 1, off] = value[:, keep]


def paged_decode_attention(q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                           block_tables: torch.Tensor, seq_lens: torch.Tensor,
                           scale: float) -> torch.Tensor:
    """q ``[B, Hq, D]`` (16-bit); key_cache/value_cache ``[N, bs, Hkv, D]``
    views; returns float32 ``[B, Hq, D]``."""
    B, Hq, D = q.shape
    bs, Hkv = key_cache.size(1), key_cache.size(2)
    G = Hq // Hkv
    out = torch.zeros((B, Hq, D), dtype=torch.float32)
    for b in range(B):
        n = int(seq_lens[b])
        if n == 0:
            continue
        ids = block_tables[b, :(n + bs - 1) // bs].long()
        k = key_cache[ids].reshape(-1, Hkv, D)[:n].float().permute(1, 2, 0)   # [Hkv, D, n]
        v = value_cache[ids].reshape(-1, Hkv, D)[:n].float().transpose(0, 1)  # [Hkv, n, D]
        qb = q[b].float().view(Hkv, G, D)
        p = torch.softmax(torch.bmm(qb, k) * scale, dim=-1)                  # [Hkv, G, n]
        out[b] = torch.bmm(p, v).reshape(Hq, D)
    return out


def swap_blocks(src_ids, dst_ids, src_pool: torch.Tensor, dst_pool: torch.Tensor) -> None:
    """``dst_pool[dst_ids[i]] = src_pool[src_ids[i]]`` for i = 0..n-1 in order
    (a repeated destination keeps the last), one block copy per pair as
    swap.cu:36-58 issues one cudaMemcpyAsync per block; host pools whose first
    axis is the block id."""
    for s, d in zip(src_ids, dst_ids):
        dst_pool[int(d)].copy_(src_pool[int(s)])
