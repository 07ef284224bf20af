"""Unified multi-model KV pool: slab geometry and compaction planning.

The reference keeps one pinned CPU pool shared by every model on a node, cut
into 1 GiB slabs that each hold blocks of a single shape; block id ``b`` of a
shape with ``bb`` bytes per block lives at byte ``b * bb`` and slab ``s``
holds ids ``[ceil(s*S/bb), floor((s+1)*S/bb))``
(aegaeon/aegaeon/block_manager.py:242-245,528-580).  Here the same scheme
describes a GPU pool that co-hosts several models' KV.

The reference never moves a KV block to compact a pool (its only compaction
slides weight slices, aegaeon/aegaeon/loader/allocator.py:288-321).  The
compaction defined here, per block shape: the live ids must end up as the
dense prefix of that shape's ordered id space; the highest live id outside the
prefix moves to the lowest hole inside it.  Sources lie outside the prefix and
destinations inside it, so the two sets are disjoint and one parallel copy
kernel (``ops.defrag_blocks``) performs every move at once.
"""
from __future__ import annotations

from typing import Iterable, List, Sequence, Tuple

import numpy as np


def slab_range(slab: int, slab_bytes: int, block_bytes: int) -> Tuple[int, int]:
    """Block ids ``[start, end)`` of a shape with ``block_bytes`` per block that
    lie wholly inside slab ``slab`` (block_manager.py:242-245)."""
    start = -(-(slab * slab_bytes) // block_bytes)
    end = ((slab + 1) * slab_bytes) // block_bytes
    return start, end


def slab_of(block: int, slab_bytes: int, block_bytes: int) -> int:
    """Slab that holds block ``block`` (block_manager.py:577-578)."""
    return block * block_bytes // slab_bytes


def plan_compaction(live_ids: Iterable[int], valid_ids: Sequence[int]
                    ) -> Tuple[np.ndarray, np.ndarray]:
    """Move list ``(src, dst)`` (int64) that packs ``live_ids`` into the first
    ``len(live)`` entries of ``valid_ids`` (the shape's id space, ascending).

    Two pointers: ``hi`` walks the live ids from the top down, skipping those
    already inside the prefix; ``lo`` walks the prefix from the bottom up,
    skipping occupied ids.  Each step pairs the current top mover with the
    current lowest hole.  Raises ``ValueError`` for duplicate or foreign ids.
    """
    valid = np.asarray(valid_ids, dtype=np.int64)
    live = np.sort(np.fromiter((int(x) for x in live_ids), dtype=np.int64))
    if live.size and np.any(live[1:] == live[:-1]):
        raise ValueError("duplicate live block id")
    if valid.size and np.any(valid[1:] <= valid[:-1]):
        raise ValueError("valid ids must be strictly ascending")
    k = live.size
    if k > valid.size:
        raise ValueError("more live blocks than the id space holds")
    pos = np.searchsorted(valid, live)
    if k and (pos.max() >= valid.size or np.any(valid[pos] != live)):
        raise ValueError("a live block id is outside the shape's id space")
    # live[i] sits at index pos[i] of the id space; prefix = indices [0, k)
    occupied = np.zeros(k, dtype=bool)
    inside = pos < k
    occupied[pos[inside]] = True
    holes = valid[:k][~occupied]           # ascending
    movers = live[~inside][::-1]           # descending
    assert holes.size == movers.size
    return movers.copy(), holes.copy()


def remap_tables(tables: Sequence[Sequence[int]], src: Sequence[int],
                 dst: Sequence[int]) -> List[List[int]]:
    """Block tables after the moves ``src[i] -> dst[i]``."""
    mp = {int(s): int(d) for s, d in zip(src, dst)}
    return [[mp.get(int(b), int(b)) for b in t] for t in tables]
