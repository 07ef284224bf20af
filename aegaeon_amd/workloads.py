"""KV geometries and seeded synthetic workloads for the data path.

Geometry follows the reference: a KV block holds ``BLOCK_SIZE = 16`` tokens of
every layer, shaped ``(L, 2, 16, Hkv, D)`` (aegaeon/aegaeon/config.py:13,
256-271); the GPU cache is ``[N, *block_shape]`` (worker.py:389-395).

The generators use ``numpy.random.default_rng(seed)``; a lognormal length with
arithmetic mean m and sigma s uses ``mu = ln m - s^2/2``, rounded and clipped.
Block tables are a seeded permutation of the pool, split per sequence, which
emulates the scattered tables the reference's FIFO free lists produce over time
(aegaeon/aegaeon/block_manager.py:525-526,703).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Sequence, Tuple

import numpy as np

BLOCK_SIZE = 16


@dataclass(frozen=True)
class KVGeometry:
    """Per-model KV block geometry (kv heads per GPU at tp=1)."""
    name: str
    n_layers: int
    n_kv_heads: int
    head_dim: int
    n_q_heads: int
    dtype: str  # "bf16" | "fp16"
    block_size: int = BLOCK_SIZE

    @property
    def elem_bytes(self) -> int:
        return 2

    @property
    def block_shape(self) -> Tuple[int, ...]:
        return (self.n_layers, 2, self.block_size, self.n_kv_heads, self.head_dim)

    @property
    def row_elems(self) -> int:
        return self.n_kv_heads * self.head_dim

    @property
    def block_elems(self) -> int:
        return int(np.prod(self.block_shape))

    @property
    def block_bytes(self) -> int:
        return self.block_elems * self.elem_bytes

    @property
    def layer_stride(self) -> int:  # elements
        return 2 * self.block_size * self.row_elems

    @property
    def kv_stride(self) -> int:  # elements
        return self.block_size * self.row_elems

    @property
    def bytes_per_token(self) -> int:
        return 2 * self.n_layers * self.row_elems * self.elem_bytes


TINY = KVGeometry("tiny-1L-2H-64D", 1, 2, 64, 2, "fp16")
QWEN25_7B = KVGeometry("Qwen2.5-7B", 28, 4, 128, 28, "bf16")
YI15_9B = KVGeometry("Yi-1.5-9B", 48, 4, 128, 32, "bf16")
LLAMA2_13B = KVGeometry("Llama-2-13B", 40, 40, 128, 40, "fp16")


def lognormal_lengths(rng: np.random.Generator, n: int, mean: float, sigma: float,
                      lo: int, hi: int) -> np.ndarray:
    mu = math.log(mean) - sigma * sigma / 2
    return np.clip(np.rint(rng.lognormal(mu, sigma, size=n)), lo, hi).astype(np.int64)


def split_tables(ids: np.ndarray, counts: Sequence[int]) -> List[List[int]]:
    out, o = [], 0
    for c in counts:
        out.append([int(x) for x in ids[o:o + c]])
        o += c
    return out


def slot_mapping_for(block_tables: Sequence[Sequence[int]], positions: Sequence[int],
                     block_size: int = BLOCK_SIZE) -> np.ndarray:
    """Slot of the token at ``positions[b]`` of each sequence:
    ``block_table[p // 16] * 16 + p % 16`` (aegaeon/aegaeon/worker.py:628-633)."""
    return np.asarray([bt[p // block_size] * block_size + p % block_size
                       for bt, p in zip(block_tables, positions)], dtype=np.int64)


def padded_tables(block_tables: Sequence[Sequence[int]], width: int = 0, pad: int = 0) -> np.ndarray:
    """int32 ``[B, width]`` padded with ``pad`` (0 in the reference,
    worker.py:640-646)."""
    w = max(width, max((len(t) for t in block_tables), default=0))
    out = np.full((len(block_tables), w), pad, dtype=np.int32)
    for i, t in enumerate(block_tables):
        out[i, :len(t)] = t
    return out


@dataclass
class DecodeBatch:
    """One decode step: sequence b holds ``context_lens[b]`` cached tokens and
    appends one at position ``context_lens[b]`` (seq_len = context_len + 1)."""
    geometry: KVGeometry
    context_lens: np.ndarray
    block_tables: List[List[int]]
    n_pool_blocks: int
    seed: int

    @property
    def batch(self) -> int:
        return len(self.context_lens)

    @property
    def seq_lens(self) -> np.ndarray:
        return self.context_lens + 1

    def slot_mapping(self) -> np.ndarray:
        return slot_mapping_for(self.block_tables, self.context_lens, self.geometry.block_size)

    def padded_tables(self) -> np.ndarray:
        return padded_tables(self.block_tables)

    @property
    def n_blocks_used(self) -> int:
        return sum(len(t) for t in self.block_tables)

    def append_bytes(self) -> int:
        """Algorithmic bytes of one all-layer append: read K and V, write the
        cache, read the slots."""
        g = self.geometry
        return 2 * self.batch * g.n_layers * 2 * g.row_elems * g.elem_bytes + 8 * self.batch

    def attention_bytes(self, seq_lens: np.ndarray | None = None) -> int:
        """Per-layer algorithmic bytes of decode attention: K and V of every
        cached token, q and out, the block-table entries read, seq_lens."""
        g = self.geometry
        sl = self.seq_lens if seq_lens is None else seq_lens
        kv = int(sl.sum()) * 2 * g.row_elems * g.elem_bytes
        qo = 2 * self.batch * g.n_q_heads * g.head_dim * g.elem_bytes
        bt = 4 * int(sum(-(-int(x) // g.block_size) for x in sl))
        return kv + qo + bt + 4 * self.batch


def _decode_batch(geom: KVGeometry, context_lens: np.ndarray, rng: np.random.Generator,
                  pool_factor: float, seed: int, n_pool: int | None = None) -> DecodeBatch:
    need = [-(-(int(c) + 1) // geom.block_size) for c in context_lens]
    total = int(sum(need))
    pool = int(n_pool) if n_pool is not None else int(math.ceil(pool_factor * total))
    if total > pool:
        raise ValueError(f"pool of {pool} blocks cannot hold {total}")
    ids = rng.permutation(pool)[:total]
    return DecodeBatch(geom, context_lens.astype(np.int64), split_tables(ids, need), pool, seed)


def tiny_batch(seed: int = 0) -> DecodeBatch:
    """1 layer, 2 KV heads, D 64, fp16, 8 sequences with context lengths
    uniform in [1, 128], blocks from a permutation of a 64-block pool."""
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1, 129, size=8).astype(np.int64)
    return _decode_batch(TINY, ctx, rng, 1.0, seed, n_pool=64)


def qwen_append_batch(seed: int = 0, batch: int = 256) -> DecodeBatch:
    """Qwen2.5-7B decode-step append: 256 sequences, context lengths
    lognormal(mean 600, sigma 1) clipped to [16, 4096], pool = 2x need."""
    rng = np.random.default_rng(seed)
    ctx = lognormal_lengths(rng, batch, 600.0, 1.0, 16, 4096)
    return _decode_batch(QWEN25_7B, ctx, rng, 2.0, seed)


def successive_step_slots(wb: DecodeBatch, n_steps: int) -> np.ndarray:
    """Slot mappings ``[n_steps, B]`` of ``n_steps`` successive decode steps of
    ``wb``: step r appends position ``context_len + r``.  Blocks that the
    longer sequences need are taken, in order, from the pool ids no table
    holds (tables grow at the tail, block_manager.py:651-694)."""
    bs = wb.geometry.block_size
    used = {b for t in wb.block_tables for b in t}
    spare = iter(b for b in range(wb.n_pool_blocks) if b not in used)
    tables = [list(t) for t in wb.block_tables]
    out = np.empty((n_steps, wb.batch), dtype=np.int64)
    for r in range(n_steps):
        for i, c in enumerate(wb.context_lens):
            pos = int(c) + r
            while len(tables[i]) <= pos // bs:
                tables[i].append(next(spare))
            out[r, i] = tables[i][pos // bs] * bs + pos % bs
    return out


def qwen_attention_batch(seed: int = 0, batch: int = 128) -> DecodeBatch:
    """Qwen2.5-7B paged decode attention: 128 sequences whose seq_len (cached
    tokens including the current one) is lognormal(mean 1500, sigma 1) clipped
    to [16, 8192]; pool = 2x need.  context_lens = seq_len - 1."""
    rng = np.random.default_rng(seed)
    sl = lognormal_lengths(rng, batch, 1500.0, 1.0, 16, 8192)
    return _decode_batch(QWEN25_7B, sl - 1, rng, 2.0, seed)


@dataclass
class SwapWorkload:
    """Llama-2-13B swap-out/swap-in: ``n_seqs`` sequences of ``seq_len`` tokens
    with scattered GPU blocks; swap out to CPU blocks 0..n-1 (consecutive ids,
    as a fresh slab hands them out, block_manager.py:574-580), then swap back in
    to a disjoint, seeded random set of free GPU blocks."""
    geometry: KVGeometry
    block_tables: List[List[int]]
    cpu_ids: List[int]
    swap_in_ids: List[int]
    n_pool_blocks: int

    @property
    def gpu_ids(self) -> List[int]:
        return [b for t in self.block_tables for b in t]

    @property
    def n_blocks(self) -> int:
        return len(self.cpu_ids)

    def pack_bytes(self) -> int:
        return 2 * self.n_blocks * self.geometry.block_bytes + 8 * self.n_blocks


def llama_swap_workload(seed: int = 0, n_seqs: int = 32, seq_len: int = 2048) -> SwapWorkload:
    geom = LLAMA2_13B
    rng = np.random.default_rng(seed)
    per = -(-seq_len // geom.block_size)
    n = n_seqs * per
    pool = 2 * n
    perm = rng.permutation(pool)
    tables = split_tables(perm[:n], [per] * n_seqs)
    free = perm[n:].copy()
    rng.shuffle(free)
    return SwapWorkload(geom, tables, list(range(n)), [int(x) for x in free[:n]], pool)


# --------------------------------------------------------------------------
# Unified multi-model pool (slabs of one block shape each)
# --------------------------------------------------------------------------
@dataclass
class UnifiedPoolWorkload:
    """A byte pool of ``n_slabs`` slabs of ``slab_bytes``; each slab holds
    blocks of one model's shape (the reference's CPU slab scheme,
    block_manager.py:186-199,242-245, applied to the GPU pool).  Block id b of
    a shape with ``bb`` bytes per block lives at byte ``b * bb``; slab s holds
    ids ``[ceil(s*S/bb), floor((s+1)*S/bb))``."""
    slab_bytes: int
    n_slabs: int
    geometries: Dict[str, KVGeometry]
    slab_owner: List[str]                       # slab -> model name
    tables: Dict[str, List[List[int]]]          # model -> per-sequence block tables
    yi_context_lens: np.ndarray                 # the decoding model's batch
    decode_model: str = "Yi-1.5-9B"

    @property
    def pool_bytes(self) -> int:
        return self.slab_bytes * self.n_slabs

    def slab_range(self, slab: int, bb: int) -> Tuple[int, int]:
        return (-(-(slab * self.slab_bytes) // bb), ((slab + 1) * self.slab_bytes) // bb)

    def valid_ids(self, model: str) -> List[int]:
        bb = self.geometries[model].block_bytes
        out: List[int] = []
        for s, owner in enumerate(self.slab_owner):
            if owner == model:
                a, b = self.slab_range(s, bb)
                out.extend(range(a, b))
        return out


def unified_pool_workload(seed: int = 0, slab_bytes: int = 1 << 30) -> UnifiedPoolWorkload:
    """Yi-1.5-9B decode batch (64 sequences, context lengths lognormal(mean
    1000, sigma 1) clipped to [16, 4096]) in a pool that co-hosts Qwen2.5-7B and
    Llama-2-13B KV; every model's slabs are 50% occupied by randomly placed live
    blocks.  Slabs are assigned to models in a seeded random order."""
    rng = np.random.default_rng(seed)
    geoms = {g.name: g for g in (YI15_9B, QWEN25_7B, LLAMA2_13B)}
    ctx = lognormal_lengths(rng, 64, 1000.0, 1.0, 16, 4096)
    yi_need = [-(-(int(c) + 1) // YI15_9B.block_size) for c in ctx]
    per_slab = {n: slab_bytes // g.block_bytes for n, g in geoms.items()}
    n_slabs = {
        YI15_9B.name: -(-2 * sum(yi_need) // per_slab[YI15_9B.name]),
        QWEN25_7B.name: 8,
        LLAMA2_13B.name: 24,
    }
    owners = [name for name, k in n_slabs.items() for _ in range(k)]
    owners = [owners[i] for i in rng.permutation(len(owners))]
    wl = UnifiedPoolWorkload(slab_bytes, len(owners), geoms, owners, {}, ctx)
    for name, g in geoms.items():
        valid = np.asarray(wl.valid_ids(name), dtype=np.int64)
        if name == YI15_9B.name:
            need = yi_need
        else:
            live_n = len(valid) // 2
            seq_blocks = 128 if name == QWEN25_7B.name else 16
            need = [seq_blocks] * (live_n // seq_blocks)
        total = int(sum(need))
        if total > len(valid) // 2 + 1:
            raise ValueError(f"{name}: {total} live blocks exceed 50% of {len(valid)}")
        live = rng.permutation(valid)[:total]
        wl.tables[name] = split_tables(live, need)
    return wl


def pinnable_blocks(block_bytes: int, want: int, reserve: int = 32 << 30) -> int:
    """How many blocks of ``block_bytes`` a pinned host pool on this host may
    hold, up to ``want``: torch's pinned allocator rounds a request up to a
    power of two, and the pool takes at most half of MemAvailable less
    ``reserve``.  Halves ``want`` until it fits (0 when nothing does)."""
    avail = 0
    try:
        with open("/proc/meminfo") as f:
            for line in f:
                if line.startswith("MemAvailable:"):
                    avail = int(line.split()[1]) * 1024
    except OSError:
        pass
    budget = (avail - reserve) // 2
    n = want
    while n > 0 and (1 << (n * block_bytes - 1).bit_length()) > budget:
        n //= 2
    return n

