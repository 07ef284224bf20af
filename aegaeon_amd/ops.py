"""Block-level KV movement with the reference's op surface.

``swap`` is a drop-in for ``aegaeon.ops.swap`` (aegaeon/ops/ops.cpp:4-5,
aegaeon/ops/swap.cu:25-59): same arguments, same meaning, the work is enqueued
on the *current* torch stream (swap.cu:32) and nothing is returned.  It differs
in four documented ways: the bytes per block come from the tensor's element
size instead of a hard-coded 2 (identical for the fp16/bf16 caches the
reference uses), ids are range-checked, duplicate destination ids raise
instead of silently racing, and a swap space that is not pinned raises instead
of silently copying synchronously.  Errors raise :class:`AegkvError`, the analogue of
the reference's ``CUDART_CHECK`` (aegaeon/aegaeon/cuda_wrapper.py:152-155).

PyTorch owns every buffer; the HIP kernels run through the C ABI of
``libaegkv.so``.
"""
from __future__ import annotations

import ctypes
import os
import threading
from typing import Dict, Optional, Sequence, Tuple, Union

import numpy as np
import torch

from . import _lib

IdList = Union[Sequence[int], np.ndarray, torch.Tensor]

# Default capacity of the per-stream staging buffer used by swap() when
# staging="auto" (one buffer per (device, stream): the swap-in and swap-out
# streams run concurrently and must not share it).
STAGING_BYTES = int(os.environ.get("AEGKV_SWAP_STAGING_MB", "256")) << 20

_staging: Dict[Tuple[int, int], torch.Tensor] = {}
_staging_lock = threading.Lock()


def _ids(x: Optional[IdList]) -> Tuple[Optional[np.ndarray], int]:
    if x is None:
        return None, 0
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    a = np.ascontiguousarray(np.asarray(x, dtype=np.int64).reshape(-1))
    return a, int(a.size)


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(t: torch.Tensor, name: str, device: Optional[torch.device] = None) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a GPU tensor")
    if device is not None and t.device != device:
        raise ValueError(f"{name} lives on {t.device}, the call on {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def block_bytes_of(pool: torch.Tensor) -> int:
    """Bytes of one block of a pool whose first axis is the block id."""
    if pool.dim() == 0 or pool.size(0) == 0:
        raise ValueError("pool must have a non-empty block axis")
    return pool.numel() * pool.element_size() // pool.size(0)


def _num_blocks(pool: torch.Tensor, bb: int) -> int:
    return pool.numel() * pool.element_size() // bb


def _staging_for(device: torch.device, stream: int, need: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _staging_lock:
        buf = _staging.get(key)
        if buf is None or buf.numel() < need:
            buf = torch.empty(max(need, STAGING_BYTES), dtype=torch.uint8, device=device)
            _staging[key] = buf
        return buf


def swap(source_block_ids: IdList, target_block_ids: IdList, is_swap_in: bool,
         kv_cache: torch.Tensor, kv_swap: torch.Tensor,
         staging: Union[None, str, torch.Tensor] = "auto",
         bounce: Optional[torch.Tensor] = None) -> None:
    """Copy block ``source_block_ids[i]`` to ``target_block_ids[i]`` between
    the GPU cache and the CPU swap space, CPU->GPU when ``is_swap_in``.

    ``kv_cache``: contiguous GPU tensor ``[N_gpu, *block_shape]``;
    ``kv_swap``: contiguous CPU tensor ``[N_cpu, *block_shape]`` or flat,
    pinned (the reference pins its swap space, worker.py:130-147), or
    pageable together with ``bounce``: the reference's shared file mapping
    where it cannot be page-locked (:func:`aegaeon_amd.swap_pool.init_cpu_cache`),
    reached through the pinned uint8 ``bounce`` buffer
    (aegkv_swap_blocks_bounced).  A pageable swap space without a bounce
    buffer is rejected: every DMA would silently become a blocking copy.
    ``staging``: "auto" packs scattered GPU blocks through a per-stream device
    buffer so that each run of consecutive CPU ids is a single DMA; None issues
    one DMA per run of consecutive id pairs; a GPU uint8 tensor is used as the
    staging buffer directly.  The bounced path always stages.
    """
    _require_device(kv_cache, "kv_cache")
    if kv_swap.is_cuda or not kv_swap.is_contiguous():
        raise ValueError("kv_swap must be a contiguous CPU tensor")
    pinned = kv_swap.is_pinned()
    if not pinned and bounce is None:
        raise ValueError("kv_swap must be pinned host memory (torch pin_memory / hipHostMalloc), "
                         "or pageable with a pinned bounce buffer: a pageable swap space makes "
                         "every copy synchronous")
    if bounce is not None and (bounce.is_cuda or not bounce.is_pinned()
                               or not bounce.is_contiguous()):
        raise ValueError("bounce must be a contiguous pinned CPU tensor")
    src, n = _ids(source_block_ids)
    dst, n2 = _ids(target_block_ids)
    if n != n2:
        raise ValueError("source_block_ids and target_block_ids differ in length")
    if n == 0:
        return
    bb = block_bytes_of(kv_cache)
    n_dev = kv_cache.size(0)
    n_host = kv_swap.numel() * kv_swap.element_size() // bb
    device = kv_cache.device
    with torch.cuda.device(device):
        stream = _stream(device)
        if isinstance(staging, str):
            if staging != "auto":
                raise ValueError("staging must be 'auto', None or a tensor")
            stg = _staging_for(device, stream, bb)
        else:
            stg = staging
            if stg is not None and (not stg.is_cuda or stg.device != device):
                raise ValueError(f"staging must be a GPU tensor on {device}")
        if bounce is not None and not pinned and stg is None:
            stg = _staging_for(device, stream, bb)
        stg_ptr, stg_bytes = (None, 0) if stg is None else (stg.data_ptr(), stg.numel() * stg.element_size())
        if pinned:
            rc = _lib.load().aegkv_swap_blocks(
                _ptr(src), _ptr(dst), n, 1 if is_swap_in else 0, kv_cache.data_ptr(), n_dev,
                kv_swap.data_ptr(), n_host, bb, stg_ptr, stg_bytes, stream)
        else:
            rc = _lib.load().aegkv_swap_blocks_bounced(
                _ptr(src), _ptr(dst), n, 1 if is_swap_in else 0, kv_cache.data_ptr(), n_dev,
                kv_swap.data_ptr(), n_host, bb, stg_ptr, stg_bytes, bounce.data_ptr(),
                bounce.numel() * bounce.element_size(), stream)
    _lib.check(rc, "swap")


def copy_blocks(src_pool: torch.Tensor, dst_pool: torch.Tensor, src_ids: Optional[IdList],
                dst_ids: Optional[IdList], block_bytes: Optional[int] = None) -> None:
    """``dst_pool[dst_ids[i]] <- src_pool[src_ids[i]]`` on the GPU (None ids
    = identity; with both None, every block of the smaller pool is copied and
    no id list is uploaded).  Same-pool moves require disjoint src/dst sets."""
    _require_device(src_pool, "src_pool")
    _require_device(dst_pool, "dst_pool", src_pool.device)
    bb = block_bytes or block_bytes_of(src_pool)
    s, ns = _ids(src_ids)
    d, nd = _ids(dst_ids)
    if s is not None and d is not None and ns != nd:
        raise ValueError("src_ids and dst_ids differ in length")
    if s is None and d is None:
        n = min(_num_blocks(src_pool, bb), _num_blocks(dst_pool, bb))
    else:
        n = ns if s is not None else nd
    with torch.cuda.device(src_pool.device):
        rc = _lib.load().aegkv_copy_blocks(
            src_pool.data_ptr(), _num_blocks(src_pool, bb), dst_pool.data_ptr(),
            _num_blocks(dst_pool, bb), _ptr(s), _ptr(d), n, bb, _stream(src_pool.device))
    _lib.check(rc, "copy_blocks")


def pack_blocks(pool: torch.Tensor, ids: IdList, out: Optional[torch.Tensor] = None,
                block_bytes: Optional[int] = None) -> torch.Tensor:
    """Gather blocks ``pool[ids]`` into a contiguous staging tensor
    (``[n, *pool.shape[1:]]``, or ``out``)."""
    _require_device(pool, "pool")
    bb = block_bytes or block_bytes_of(pool)
    a, n = _ids(ids)
    if out is None:
        if block_bytes is None:
            out = torch.empty((n, *pool.shape[1:]), dtype=pool.dtype, device=pool.device)
        else:
            out = torch.empty(n * bb, dtype=torch.uint8, device=pool.device)
    _require_device(out, "out", pool.device)
    if out.numel() * out.element_size() < n * bb:
        raise ValueError("out is smaller than the packed blocks")
    with torch.cuda.device(pool.device):
        rc = _lib.load().aegkv_pack_blocks(pool.data_ptr(), _num_blocks(pool, bb), _ptr(a), n,
                                           out.data_ptr(), bb, _stream(pool.device))
    _lib.check(rc, "pack_blocks")
    return out


def scatter_blocks(staging: torch.Tensor, ids: IdList, pool: torch.Tensor,
                   block_bytes: Optional[int] = None) -> None:
    """``pool[ids[i]] <- staging[i]``."""
    _require_device(pool, "pool")
    _require_device(staging, "staging", pool.device)
    bb = block_bytes or block_bytes_of(pool)
    a, n = _ids(ids)
    if staging.numel() * staging.element_size() < n * bb:
        raise ValueError("staging is smaller than the scattered blocks")
    with torch.cuda.device(pool.device):
        rc = _lib.load().aegkv_scatter_blocks(staging.data_ptr(), _ptr(a), n, pool.data_ptr(),
                                              _num_blocks(pool, bb), bb, _stream(pool.device))
    _lib.check(rc, "scatter_blocks")


def defrag_blocks(pool: torch.Tensor, src_ids: IdList, dst_ids: IdList,
                  block_bytes: Optional[int] = None) -> None:
    """In-pool block moves ``pool[dst[i]] <- pool[src[i]]`` with disjoint
    src/dst sets (one parallel kernel).  ``block_bytes`` selects the block
    shape of a multi-shape byte pool."""
    _require_device(pool, "pool")
    bb = block_bytes or block_bytes_of(pool)
    s, ns = _ids(src_ids)
    d, nd = _ids(dst_ids)
    if ns != nd:
        raise ValueError("src_ids and dst_ids differ in length")
    with torch.cuda.device(pool.device):
        rc = _lib.load().aegkv_defrag_blocks(pool.data_ptr(), _num_blocks(pool, bb), _ptr(s),
                                             _ptr(d), ns, bb, _stream(pool.device))
    _lib.check(rc, "defrag_blocks")
