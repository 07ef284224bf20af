"""numpy restatement of the reference's KV-cache data path (test infrastructure).

Layout conventions follow the reference:
  * GPU KV storage is ``[N_blocks, L, 2, 16, Hkv, D]`` contiguous
    (aegaeon/aegaeon/worker.py:389-395, aegaeon/aegaeon/config.py:256-271);
  * the per-layer vLLM view is ``storage.permute(1, 2, 0, 3, 4, 5)[l][kv]``,
    i.e. ``[N, 16, Hkv, D]`` with block stride ``L*2*16*Hkv*D``
    (worker.py:419-451);
  * a block of ``block_bytes`` bytes starts at ``id * block_bytes`` in both the
    GPU pool and the CPU swap pool (aegaeon/ops/swap.cu:34,43-44,52-53).

Arrays of 16-bit floats are carried as ``uint16`` bit patterns for byte moves;
``bits_to_float`` converts bf16/fp16 patterns to float64 for attention.
"""
from __future__ import annotations

import math
from typing import List, Sequence, Tuple

import numpy as np

BLOCK_SIZE = 16  # aegaeon/aegaeon/config.py:13


# --------------------------------------------------------------------------
# a1: swap (aegaeon/ops/swap.cu:25-59)
# --------------------------------------------------------------------------
def swap_blocks(src_ids: Sequence[int], dst_ids: Sequence[int], is_swap_in: bool,
                kv_cache: np.ndarray, kv_swap: np.ndarray) -> None:
    """In-place restatement of ``swap``.

    ``kv_cache`` and ``kv_swap`` are arrays whose first axis is the block id
    (any dtype).  For each i, block ``src_ids[i]`` of the source pool is
    copied byte-for-byte to block ``dst_ids[i]`` of the destination pool, in
    order i = 0..n-1 (swap.cu:36-58); H2D when ``is_swap_in``.
    """
    cache = kv_cache.reshape(kv_cache.shape[0], -1).view(np.uint8)
    swap = kv_swap.reshape(kv_swap.shape[0], -1).view(np.uint8)
    src, dst = (swap, cache) if is_swap_in else (cache, swap)
    for s, d in zip(src_ids, dst_ids):
        dst[int(d)] = src[int(s)]


def copy_blocks(src_pool: np.ndarray, dst_pool: np.ndarray, src_ids, dst_ids) -> None:
    """dst_pool[dst_ids[i]] <- src_pool[src_ids[i]] (None = identity)."""
    n = len(src_ids) if src_ids is not None else len(dst_ids)
    s = np.arange(n) if src_ids is None else np.asarray(src_ids, dtype=np.int64)
    d = np.arange(n) if dst_ids is None else np.asarray(dst_ids, dtype=np.int64)
    src = src_pool.reshape(src_pool.shape[0], -1).view(np.uint8)
    dst = dst_pool.reshape(dst_pool.shape[0], -1).view(np.uint8)
    dst[d] = src[s]


def pack_blocks(pool: np.ndarray, ids) -> np.ndarray:
    """staging[i] <- pool[ids[i]] (the swap-out gather)."""
    return pool[np.asarray(ids, dtype=np.int64)].copy()


def scatter_blocks(staging: np.ndarray, ids, pool: np.ndarray) -> None:
    """pool[ids[i]] <- staging[i] (the swap-in scatter)."""
    pool[np.asarray(ids, dtype=np.int64)] = staging


# --------------------------------------------------------------------------
# a4: decode inputs (aegaeon/aegaeon/worker.py:554-713, utils.py:241-257)
# --------------------------------------------------------------------------
def slot_mapping(block_tables: Sequence[Sequence[int]], context_lens: Sequence[int],
                 seq_lens: Sequence[int], block_size: int = BLOCK_SIZE) -> np.ndarray:
    """``slot = block_table[i // 16] * 16 + i % 16`` for i in
    ``[context_len, seq_len)``, concatenated over requests (worker.py:628-633)."""
    out: List[int] = []
    for bt, c, s in zip(block_tables, context_lens, seq_lens):
        for i in range(c, s):
            out.append(bt[i // block_size] * block_size + i % block_size)
    return np.asarray(out, dtype=np.int64)


def pad_block_tables(tables: Sequence[Sequence[int]], pad: int = 0) -> np.ndarray:
    """int32 ``[B, max_len]`` padded with ``pad`` (0 in the reference,
    worker.py:640-646 via utils.py:241-257)."""
    max_len = max((len(t) for t in tables), default=0)
    out = np.full((len(tables), max_len), pad, dtype=np.int32)
    for i, t in enumerate(tables):
        out[i, :len(t)] = t
    return out


def prepare_model_inputs(requests, block_tables, block_size: int = BLOCK_SIZE):
    """Restatement of ``Worker._prepare_model_inputs`` (worker.py:596-676),
    host loops included: returns a dict of numpy arrays / ints with the
    reference's names and dtypes (input_tokens, input_positions, slot_mapping
    int64; block_tables, seq_lens_tensor, context_lens_tensor,
    query_start_loc, seq_start_loc int32)."""
    input_tokens, input_positions, slot_mapping = [], [], []
    seq_lens, prefill_seq_lens, decode_seq_lens, context_lens, query_lens = [], [], [], [], []
    tables = []
    num_prefills = num_prefill_tokens = num_decode_tokens = 0
    for (_, tokens, seq_len, context_len), _bt in zip(requests, block_tables):
        is_prompt = context_len == 0
        tables.append(list(_bt) if not is_prompt else [])          # worker.py:600-605
        seq_lens.append(seq_len)
        context_lens.append(context_len)
        query_lens.append(seq_len - context_len)
        input_tokens.extend(tokens)
        input_positions.extend(range(context_len, seq_len))
        if is_prompt:
            num_prefills += 1
            num_prefill_tokens += len(tokens)
            prefill_seq_lens.append(seq_len)
        else:
            num_decode_tokens += seq_len - context_len
            decode_seq_lens.append(seq_len)
        for i in range(context_len, seq_len):                        # worker.py:628-633
            slot_mapping.append(_bt[i // block_size] * block_size + i % block_size)
    width = max(len(t) for t in tables)
    padded = pad_block_tables(tables) if width else np.zeros((len(tables), 0), dtype=np.int32)
    q = np.asarray(query_lens, dtype=np.int64)
    sl = np.asarray(seq_lens, dtype=np.int32)
    return dict(
        input_tokens=np.asarray(input_tokens, dtype=np.int64),
        input_positions=np.asarray(input_positions, dtype=np.int64),
        slot_mapping=np.asarray(slot_mapping, dtype=np.int64),
        num_prefills=num_prefills, num_prefill_tokens=num_prefill_tokens,
        num_decode_tokens=num_decode_tokens, seq_lens=list(seq_lens),
        seq_lens_tensor=sl, context_lens_tensor=np.asarray(context_lens, dtype=np.int32),
        max_query_len=int(q.max()), max_prefill_seq_len=max(prefill_seq_lens, default=0),
        max_decode_seq_len=max(decode_seq_lens, default=0),
        query_start_loc=np.concatenate([[0], np.cumsum(q)]).astype(np.int32),
        seq_start_loc=np.concatenate([[0], np.cumsum(sl)]).astype(np.int32),
        block_tables=padded,
    )


# --------------------------------------------------------------------------
# a5: append (EXT vLLM reshape_and_cache_flash, reached from worker.py:517-523)
# --------------------------------------------------------------------------
def reshape_and_cache_flash(key: np.ndarray, value: np.ndarray, key_cache: np.ndarray,
                            value_cache: np.ndarray, slots: np.ndarray) -> None:
    """For token t with slot s >= 0: ``key_cache[s // bs, s % bs] = key[t]``,
    likewise V.  ``key_cache``: ``[N, bs, Hkv, D]`` (may be a strided view)."""
    bs = key_cache.shape[1]
    for t, s in enumerate(np.asarray(slots, dtype=np.int64)):
        if s < 0:
            continue
        key_cache[s // bs, s % bs] = key[t]
        value_cache[s // bs, s % bs] = value[t]


def append_layers(key: np.ndarray, value: np.ndarray, storage: np.ndarray,
                  slots: np.ndarray) -> None:
    """Every layer of the ``[N, L, 2, bs, Hkv, D]`` storage at once:
    layer l gets ``key[l]`` / ``value[l]`` through the vLLM view."""
    view = storage.transpose(1, 2, 0, 3, 4, 5)  # [L, 2, N, bs, Hkv, D]
    for l in range(key.shape[0]):
        reshape_and_cache_flash(key[l], value[l], view[l, 0], view[l, 1], slots)


# --------------------------------------------------------------------------
# gather_tokens: de-page through block tables
# --------------------------------------------------------------------------
def gather_tokens(storage: np.ndarray, block_tables: Sequence[Sequence[int]],
                  seq_lens: Sequence[int], layers: Sequence[int] | None = None
                  ) -> Tuple[np.ndarray, np.ndarray]:
    """Returns ``out_k, out_v`` of shape ``[len(layers), sum(len), Hkv, D]``:
    token p of sequence b comes from block ``block_tables[b][p // bs]`` row
    ``p % bs``."""
    n, L, _, bs, H, D = storage.shape
    layers = list(range(L)) if layers is None else list(layers)
    total = int(sum(seq_lens))
    out_k = np.empty((len(layers), total, H, D), dtype=storage.dtype)
    out_v = np.empty_like(out_k)
    base = 0
    for b, ln in enumerate(seq_lens):
        ln = int(ln)
        if ln == 0:
            continue
        nb = -(-ln // bs)
        ids = np.asarray(block_tables[b][:nb], dtype=np.int64)
        for li, l in enumerate(layers):
            k = storage[ids, l, 0].reshape(nb * bs, H, D)[:ln]
            v = storage[ids, l, 1].reshape(nb * bs, H, D)[:ln]
            out_k[li, base:base + ln] = k
            out_v[li, base:base + ln] = v
        base += ln
    return out_k, out_v


# --------------------------------------------------------------------------
# a10: defrag (build definition; the reference compacts only weight slices,
# aegaeon/aegaeon/loader/allocator.py:288-321)
# --------------------------------------------------------------------------
def plan_defrag(live_ids: Sequence[int], valid_ids: Sequence[int]) -> Tuple[List[int], List[int]]:
    """Two-pointer compaction.  ``valid_ids`` is the ordered id space of one
    block shape (ascending); the target is its first ``|live|`` ids.  The
    highest live id outside the target moves to the lowest hole inside it.
    Returns ``(src, dst)``; src and dst are disjoint by construction."""
    live = sorted(set(int(x) for x in live_ids))
    target = list(valid_ids[:len(live)])
    tset = set(target)
    lset = set(live)
    holes = [x for x in target if x not in lset]              # ascending
    movers = sorted((x for x in live if x not in tset), reverse=True)
    assert len(holes) == len(movers)
    return movers, holes


def apply_defrag(block_tables: Sequence[Sequence[int]], src: Sequence[int],
                 dst: Sequence[int]) -> List[List[int]]:
    """Rewrite block tables through the move map src[i] -> dst[i]."""
    mp = dict(zip((int(s) for s in src), (int(d) for d in dst)))
    return [[mp.get(int(x), int(x)) for x in bt] for bt in block_tables]


# --------------------------------------------------------------------------
# a6: paged decode attention (EXT flash_attn_with_kvcache, worker.py:410-418)
# --------------------------------------------------------------------------
def bits_to_float(bits: np.ndarray, dtype: str) -> np.ndarray:
    """uint16 bit patterns of bf16/fp16 -> float64."""
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype == "bf16":
        return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    if dtype == "fp16":
        return bits.view(np.float16).astype(np.float64)
    raise ValueError(dtype)


def float_to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """float -> uint16 patterns with round-to-nearest-even."""
    x = np.asarray(x)
    if dtype == "fp16":
        return x.astype(np.float16).view(np.uint16)
    if dtype == "bf16":
        u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
        r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
        return r.astype(np.uint16)
    raise ValueError(dtype)


def paged_decode_attention(q: np.ndarray, key_cache: np.ndarray, value_cache: np.ndarray,
                           block_tables: np.ndarray, seq_lens: Sequence[int],
                           scale: float) -> np.ndarray:
    """Textbook softmax attention in float64.

    q: ``[B, Hq, D]`` float; key_cache/value_cache: ``[N, bs, Hkv, D]`` float
    views; query head h reads kv head ``h // (Hq // Hkv)``.  Tokens
    ``j < seq_lens[b]`` through ``block_tables[b][j // bs]``.
    """
    B, Hq, D = q.shape
    bs, Hkv = key_cache.shape[1], key_cache.shape[2]
    G = Hq // Hkv
    out = np.zeros((B, Hq, D), dtype=np.float64)
    for b in range(B):
        ln = int(seq_lens[b])
        if ln == 0:
            continue
        nb = -(-ln // bs)
        ids = np.asarray(block_tables[b][:nb], dtype=np.int64)
        k = key_cache[ids].reshape(nb * bs, Hkv, D)[:ln].astype(np.float64)
        v = value_cache[ids].reshape(nb * bs, Hkv, D)[:ln].astype(np.float64)
        qb = q[b].astype(np.float64).reshape(Hkv, G, D)
        s = np.einsum("hgd,thd->hgt", qb, k) * scale
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[b] = np.einsum("hgt,thd->hgd", p, v).reshape(Hq, D)
    return out


# --------------------------------------------------------------------------
# prefill: EXT flash_attn_varlen_func, the prompt run of vLLM's
# FlashAttention backend (reached from worker.py:517-523; cu_seqlens =
# seq_start_loc, worker.py:665-673)
# --------------------------------------------------------------------------
def varlen_prefill_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                             cu_seqlens: Sequence[int], scale: float,
                             causal: bool = True) -> np.ndarray:
    """Textbook softmax attention of packed sequences in float64.

    q: ``[T, Hq, D]``, k/v: ``[T, Hkv, D]`` float; sequence b is tokens
    ``cu_seqlens[b] .. cu_seqlens[b+1]``; query i of a sequence sees keys
    ``j <= i`` of it when causal, all of them otherwise; query head h reads kv
    head ``h // (Hq // Hkv)``.  Tokens outside every sequence stay 0.
    """
    T, Hq, D = q.shape
    Hkv = k.shape[1]
    G = Hq // Hkv
    out = np.zeros((T, Hq, D), dtype=np.float64)
    for b in range(len(cu_seqlens) - 1):
        s0, s1 = int(cu_seqlens[b]), int(cu_seqlens[b + 1])
        n = s1 - s0
        if n <= 0:
            continue
        # [Hkv, G, n, D] queries against [Hkv, 1, n, D] keys and values
        # (batched matrix products, so long prompts finish in seconds)
        qb = q[s0:s1].astype(np.float64).reshape(n, Hkv, G, D).transpose(1, 2, 0, 3)
        kb = k[s0:s1].astype(np.float64).transpose(1, 0, 2)[:, None]
        vb = v[s0:s1].astype(np.float64).transpose(1, 0, 2)[:, None]
        s = np.matmul(qb, kb.transpose(0, 1, 3, 2)) * scale
        if causal:
            s = np.where(np.tril(np.ones((n, n), dtype=bool)), s, -np.inf)
        s -= s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(axis=-1, keepdims=True)
        out[s0:s1] = np.matmul(p, vb).transpose(2, 0, 1, 3).reshape(n, Hq, D)
    return out
