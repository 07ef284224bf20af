"""Token-level KV ops with the vLLM 0.5.1 surface the reference reaches from
its model forward (aegaeon/aegaeon/worker.py:517-523):

* :func:`reshape_and_cache_flash` — vLLM's per-layer K/V append into the
  flash-attn cache view ``[N, 16, Hkv, D]``;
* :func:`append_kv` — the same append for every layer of the reference's
  ``[N, L, 2, 16, Hkv, D]`` storage (worker.py:389-395) in one launch;
* :func:`gather_tokens` — block-table de-page into contiguous buffers;
* :func:`flash_attn_with_kvcache` — vllm-flash-attn's paged decode call
  (selected at worker.py:410-418) for one query token per sequence;
* :func:`flash_attn_varlen_func` — vllm-flash-attn's varlen call of the
  backend's prompt run (causal attention of packed prompts).

All of them enqueue hand-written gfx950 kernels on the current torch stream.
"""
from __future__ import annotations

import math
import threading
import weakref
from typing import Dict, Optional, Sequence, Tuple

import torch

from . import _lib

_DTYPES = {torch.bfloat16: _lib.AEGKV_DTYPE_BF16, torch.float16: _lib.AEGKV_DTYPE_FP16}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _check_cache_view(c: torch.Tensor, name: str) -> None:
    """A per-layer cache view ``[N, bs, Hkv, D]`` with dense rows per block."""
    if c.dim() != 4 or not c.is_cuda:
        raise ValueError(f"{name} must be a 4-d GPU tensor [N, block_size, Hkv, D]")
    N, bs, H, D = c.shape
    if c.stride(3) != 1 or c.stride(2) != D or c.stride(1) != H * D:
        raise ValueError(f"{name}: each block must hold dense [block_size, Hkv, D] rows")


def _check_on(t: torch.Tensor, name: str, device: torch.device) -> None:
    """A metadata tensor the kernel reads must live on the kernel's GPU."""
    if not t.is_cuda or t.device != device:
        raise ValueError(f"{name} must be a GPU tensor on {device} (got {t.device})")


def _check_rows(x: torch.Tensor, name: str) -> None:
    if not x.is_cuda or x.stride(-1) != 1 or x.stride(-2) != x.size(-1):
        raise ValueError(f"{name}: rows [Hkv, D] must be dense on the GPU")


def reshape_and_cache_flash(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                            value_cache: torch.Tensor, slot_mapping: torch.Tensor,
                            kv_cache_dtype: str = "auto") -> None:
    """For token t with ``s = slot_mapping[t] >= 0``:
    ``key_cache[s // bs, s % bs] = key[t]`` and likewise for V.

    key/value: ``[T, Hkv, D]`` (token stride may exceed Hkv*D);
    key_cache/value_cache: ``[N, bs, Hkv, D]`` views with any block stride;
    slot_mapping: int64 GPU tensor ``[T]``.  Only ``kv_cache_dtype="auto"``
    (the reference's setting, aegaeon/aegaeon/models.py:384-390) is supported.
    """
    if kv_cache_dtype != "auto":
        raise NotImplementedError("only kv_cache_dtype='auto' is supported")
    _check_cache_view(key_cache, "key_cache")
    _check_cache_view(value_cache, "value_cache")
    _check_rows(key, "key")
    _check_rows(value, "value")
    if key_cache.stride(0) != value_cache.stride(0):
        raise ValueError("key_cache and value_cache must share the block stride")
    if slot_mapping.dtype != torch.int64 or not slot_mapping.is_cuda:
        raise ValueError("slot_mapping must be an int64 GPU tensor")
    for t, n in ((key, "key"), (value, "value"), (value_cache, "value_cache"),
                 (slot_mapping, "slot_mapping")):
        _check_on(t, n, key_cache.device)
    if key.dtype != key_cache.dtype or value.dtype != key_cache.dtype \
            or value_cache.dtype != key_cache.dtype or key.element_size() != 2:
        raise ValueError("key, value and the caches must share one 16-bit dtype")
    if key.dim() != 3 or value.shape != key.shape or key.shape[1:] != key_cache.shape[2:]:
        raise ValueError("key/value must be [T, Hkv, D] matching the cache view")
    T = key.size(0)
    if slot_mapping.dim() != 1 or slot_mapping.numel() < T:
        raise ValueError(f"slot_mapping must hold a slot for each of the {T} tokens")
    N, bs, H, D = key_cache.shape
    slot_mapping = slot_mapping.contiguous()
    with torch.cuda.device(key.device):
        rc = _lib.load().aegkv_kv_append(
            key.data_ptr(), value.data_ptr(), key.stride(0), value.stride(0), 0, 0,
            slot_mapping.data_ptr(), T, key_cache.data_ptr(), value_cache.data_ptr(),
            key_cache.stride(0), 0, N, 1, bs, H, D, key.element_size(), _stream(key))
    _lib.check(rc, "reshape_and_cache_flash")


def append_kv(key: torch.Tensor, value: torch.Tensor, kv_cache: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
    """Append one decode step for every layer in one launch.

    key/value: ``[L, T, Hkv, D]`` (dense rows; token and layer strides free);
    kv_cache: the reference's contiguous storage ``[N, L, 2, bs, Hkv, D]``.
    """
    if kv_cache.dim() != 6 or not kv_cache.is_contiguous() or not kv_cache.is_cuda:
        raise ValueError("kv_cache must be a contiguous GPU tensor [N, L, 2, bs, Hkv, D]")
    N, L, two, bs, H, D = kv_cache.shape
    if key.dim() != 4 or key.size(0) != L or key.shape[2:] != (H, D) or value.shape != key.shape:
        raise ValueError("key/value must be [L, T, Hkv, D] matching the cache")
    _check_rows(key, "key")
    _check_rows(value, "value")
    if slot_mapping.dtype != torch.int64 or not slot_mapping.is_cuda:
        raise ValueError("slot_mapping must be an int64 GPU tensor")
    for t, n in ((key, "key"), (value, "value"), (slot_mapping, "slot_mapping")):
        _check_on(t, n, kv_cache.device)
    if key.dtype != kv_cache.dtype or value.dtype != kv_cache.dtype or key.element_size() != 2:
        raise ValueError("key, value and kv_cache must share one 16-bit dtype")
    T = key.size(1)
    if slot_mapping.dim() != 1 or slot_mapping.numel() < T:
        raise ValueError(f"slot_mapping must hold a slot for each of the {T} tokens")
    slot_mapping = slot_mapping.contiguous()
    kv_stride = bs * H * D
    with torch.cuda.device(kv_cache.device):
        base = kv_cache.data_ptr()
        rc = _lib.load().aegkv_kv_append(
            key.data_ptr(), value.data_ptr(), key.stride(1), value.stride(1), key.stride(0),
            value.stride(0), slot_mapping.data_ptr(), T, base,
            base + kv_stride * kv_cache.element_size(), kv_cache.stride(0), kv_cache.stride(1), N,
            L, bs, H, D, kv_cache.element_size(), _stream(kv_cache))
    _lib.check(rc, "append_kv")


def gather_tokens(kv_cache: torch.Tensor, block_tables: torch.Tensor, seq_lens: torch.Tensor,
                  total_tokens: int, max_seq_len: int, layers: Optional[Tuple[int, int]] = None,
                  cu_seqlens: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """De-page sequences: returns ``(out_k, out_v)`` of shape
    ``[n_layers, total_tokens, Hkv, D]`` with sequence b's tokens at
    ``cu_seqlens[b] : cu_seqlens[b] + seq_lens[b]``.

    kv_cache: storage ``[N, L, 2, bs, Hkv, D]``; block_tables int32
    ``[B, max_blocks]`` (0-padded like worker.py:640-646); seq_lens int32 [B];
    total_tokens and max_seq_len: host-side sum and maximum of seq_lens;
    layers: ``(first, count)`` (default all).
    """
    if kv_cache.dim() != 6 or not kv_cache.is_contiguous() or not kv_cache.is_cuda:
        raise ValueError("kv_cache must be a contiguous GPU tensor [N, L, 2, bs, Hkv, D]")
    N, L, _, bs, H, D = kv_cache.shape
    first, count = layers if layers is not None else (0, L)
    if not (0 <= first and first + count <= L and count > 0):
        raise ValueError("layer range out of bounds")
    dev = kv_cache.device
    _check_on(block_tables, "block_tables", dev)
    _check_on(seq_lens, "seq_lens", dev)
    if block_tables.dim() != 2 or seq_lens.dim() != 1 or block_tables.size(0) != seq_lens.numel():
        raise ValueError("block_tables must be [B, max_blocks] and seq_lens [B]")
    bt = _int32_dense(block_tables)
    sl = _int32_dense(seq_lens)
    if cu_seqlens is None:
        cu_seqlens = torch.zeros(sl.numel() + 1, dtype=torch.int32, device=dev)
        torch.cumsum(sl, 0, dtype=torch.int32, out=cu_seqlens[1:])
    else:
        _check_on(cu_seqlens, "cu_seqlens", dev)
        if cu_seqlens.dtype != torch.int32 or cu_seqlens.dim() != 1 \
                or not cu_seqlens.is_contiguous() or cu_seqlens.numel() != sl.numel() + 1:
            raise ValueError("cu_seqlens must be a contiguous int32 GPU tensor [B + 1]")
    out_k = torch.empty((count, total_tokens, H, D), dtype=kv_cache.dtype, device=kv_cache.device)
    out_v = torch.empty_like(out_k)
    if total_tokens == 0:
        return out_k, out_v
    es = kv_cache.element_size()
    with torch.cuda.device(kv_cache.device):
        base = kv_cache.data_ptr() + first * kv_cache.stride(1) * es
        rc = _lib.load().aegkv_gather_tokens(
            base, base + bs * H * D * es, kv_cache.stride(0), kv_cache.stride(1), N,
            bt.data_ptr(), bt.size(1), sl.data_ptr(), cu_seqlens.data_ptr(), sl.numel(),
            max_seq_len, out_k.data_ptr(), out_v.data_ptr(), total_tokens, total_tokens * H * D,
            count, bs, H, D, es, _stream(kv_cache))
    _lib.check(rc, "gather_tokens")
    return out_k, out_v


def _gpu(device) -> torch.device:
    """``device`` as a GPU device with an index (None: the current GPU)."""
    if device is None:
        return torch.device("cuda", torch.cuda.current_device())
    dev = torch.device(device)
    if dev.type != "cuda":
        raise ValueError(f"the attention workspace lives on a GPU, not on {dev}")
    return dev if dev.index is not None else torch.device("cuda", torch.cuda.current_device())


def attention_workspace_bytes(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int,
                              max_seq_len: int, dtype: torch.dtype = torch.bfloat16,
                              n_workgroups: int = 0, device=None) -> int:
    """Workspace bytes of one attention call of these sizes on ``device``
    (the default workgroup count depends on the device)."""
    if dtype not in _DTYPES:
        raise ValueError("dtype must be bfloat16 or float16")
    dev = _gpu(device)
    with torch.cuda.device(dev):
        n = _lib.load().aegkv_paged_decode_attention_workspace_size(
            batch, n_q_heads, n_kv_heads, head_dim, max_seq_len, _DTYPES[dtype], n_workgroups)
    if n < 0:
        _lib.check(int(n), "attention_workspace_bytes")
    return int(n)


def attention_workspace(batch: int, n_q_heads: int, n_kv_heads: int, head_dim: int,
                        max_seq_len: int, dtype: torch.dtype = torch.bfloat16,
                        n_workgroups: int = 0, device=None) -> Optional[torch.Tensor]:
    """A device workspace large enough for every call of these sizes (None
    when the call needs none); reusable by consecutive calls on one stream,
    calls that may overlap (other streams) need their own."""
    dev = _gpu(device)
    n = attention_workspace_bytes(batch, n_q_heads, n_kv_heads, head_dim, max_seq_len, dtype,
                                  n_workgroups, dev)
    if n == 0:
        return None
    return torch.empty(n, dtype=torch.uint8, device=dev)


# Workspaces kept per (device, stream) for calls that bring none.
_workspaces: Dict[Tuple[int, int], torch.Tensor] = {}
_ws_lock = threading.Lock()


def _cached_workspace(device: torch.device, stream: int, nbytes: int) -> torch.Tensor:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
            _workspaces[key] = ws
        return ws


def _int32_dense(t: torch.Tensor) -> torch.Tensor:
    return t if (t.dtype == torch.int32 and t.is_contiguous()) else t.to(torch.int32).contiguous()


class DecodePlan:
    """The attention's work split for one decode step (aegkv_paged_decode_plan):
    which blocks each workgroup takes and the block ids in that order, built
    once from the step's block tables and lengths and passed to every layer's
    :func:`paged_decode_attention` (``plan=``).  The tables and lengths must
    not change while the plan is in use; the plan keeps references to them.
    Batches above 2048 sequences are not planned (AegkvError)."""

    def __init__(self, block_tables: torch.Tensor, seq_lens: torch.Tensor, max_seq_len: int,
                 n_kv_heads: int, n_workgroups: int = 0):
        if not block_tables.is_cuda or not seq_lens.is_cuda or block_tables.dim() != 2 \
                or block_tables.device != seq_lens.device:
            raise ValueError("block_tables [B, max_blocks] and seq_lens [B] must be tensors on "
                             "one GPU")
        self.block_tables = _int32_dense(block_tables)
        self.seq_lens = _int32_dense(seq_lens)
        self.batch = int(self.seq_lens.numel())
        if self.block_tables.size(0) != self.batch:
            raise ValueError("block_tables and seq_lens disagree on the batch")
        self.max_seq_len = int(max_seq_len)
        self.n_kv_heads = int(n_kv_heads)
        self.n_workgroups = int(n_workgroups)
        dev = self.seq_lens.device
        lib = _lib.load()
        with torch.cuda.device(dev):
            n = lib.aegkv_paged_decode_plan_size(self.batch, self.n_kv_heads, self.max_seq_len,
                                                  self.n_workgroups)
            if n < 0:
                _lib.check(int(n), "decode_plan")
            self.buffer = torch.empty(max(int(n), 1), dtype=torch.uint8, device=dev)
            self.nbytes = int(n)
            stream = torch.cuda.current_stream(dev)
            rc = lib.aegkv_paged_decode_plan(
                self.block_tables.data_ptr(), self.block_tables.size(1), self.seq_lens.data_ptr(),
                self.batch, self.max_seq_len, self.n_kv_heads, self.n_workgroups,
                self.buffer.data_ptr(), self.nbytes, stream.cuda_stream)
            _lib.check(rc, "decode_plan")
            # Calls on another stream wait for the build (wait_for_build).
            self.stream = stream
            self.built = torch.cuda.Event()
            self.built.record(stream)

    def wait_for_build(self, stream: torch.cuda.Stream) -> None:
        """Order ``stream`` after the plan's build (a no-op on the build stream);
        the plan's memory is then also kept from reuse until ``stream`` is done
        with it."""
        if stream != self.stream:
            stream.wait_event(self.built)
            for t in (self.buffer, self.block_tables, self.seq_lens):
                t.record_stream(stream)


def paged_decode_attention(q: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                           block_tables: Optional[torch.Tensor], seq_lens: Optional[torch.Tensor],
                           scale: float, max_seq_len: int, out: Optional[torch.Tensor] = None,
                           n_workgroups: int = 0,
                           workspace: Optional[torch.Tensor] = None,
                           plan: Optional[DecodePlan] = None,
                           key: Optional[torch.Tensor] = None,
                           value: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Paged GQA decode attention: ``q [B, Hq, D]`` against per-layer cache
    views ``[N, 16, Hkv, D]``; returns ``out [B, Hq, D]`` in q's dtype.
    ``n_workgroups`` = 0 spreads the batch over one workgroup per CU; a
    positive count forces that many (same result).  ``workspace``: from
    :func:`attention_workspace` (reusable on one stream); by default a cached
    one per (device, stream).  ``plan``: a :class:`DecodePlan` of this step's
    tables and lengths (then ``block_tables``/``seq_lens`` may be None, or
    must be the tensors it was built from); the result is identical.
    ``key``/``value`` ``[B, Hkv, D]``: append them first, in the same call
    (aegkv_paged_decode_attention_append): ``seq_lens[b]`` counts the new
    token, which lands at position ``seq_lens[b] - 1`` of sequence b's table
    (the slot the reference's slot mapping gives it); the output and the cache
    equal those of :func:`reshape_and_cache_flash` followed by this call
    without ``key``/``value``, bit for bit, at the cost of the attention's
    launches alone."""
    if plan is not None:
        if plan.buffer.device != q.device:
            raise ValueError(f"the plan lives on {plan.buffer.device}, the call on {q.device}")
        for given, held, name in ((block_tables, plan.block_tables, "block_tables"),
                                  (seq_lens, plan.seq_lens, "seq_lens")):
            if given is not None and given.data_ptr() != held.data_ptr():
                raise ValueError(f"{name} is not the tensor the plan was built from")
        if (max_seq_len != plan.max_seq_len or n_workgroups != plan.n_workgroups
                or q.size(0) != plan.batch or key_cache.size(2) != plan.n_kv_heads):
            raise ValueError("the plan was built for another batch, max_seq_len, kv-head count "
                             "or workgroup count")
        block_tables, seq_lens = plan.block_tables, plan.seq_lens
    if q.dim() != 3 or q.stride(2) != 1 or q.stride(1) != q.size(2) or not q.is_cuda:
        raise ValueError("q must be a GPU tensor [B, Hq, D] with dense heads")
    _check_cache_view(key_cache, "key_cache")
    _check_cache_view(value_cache, "value_cache")
    dev = q.device
    _check_on(key_cache, "key_cache", dev)
    _check_on(value_cache, "value_cache", dev)
    if block_tables is None or seq_lens is None:
        raise ValueError("block_tables and seq_lens are required without a plan")
    _check_on(block_tables, "block_tables", dev)
    _check_on(seq_lens, "seq_lens", dev)
    if block_tables.dim() != 2 or seq_lens.dim() != 1 or block_tables.size(0) != q.size(0) \
            or seq_lens.numel() != q.size(0):
        raise ValueError("block_tables must be [B, max_blocks] and seq_lens [B] for q's batch")
    if key_cache.stride(0) != value_cache.stride(0):
        raise ValueError("key_cache and value_cache must share the block stride")
    if q.dtype not in _DTYPES or key_cache.dtype != q.dtype or value_cache.dtype != q.dtype:
        raise ValueError("q, key_cache and value_cache must share a bf16/fp16 dtype")
    B, Hq, D = q.shape
    N, bs, Hkv, _ = key_cache.shape
    bt = _int32_dense(block_tables)
    sl = _int32_dense(seq_lens)
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    elif out.shape != (B, Hq, D) or out.stride(2) != 1 or out.stride(1) != D:
        raise ValueError("out must be [B, Hq, D] with dense heads")
    elif out.dtype != q.dtype:
        raise ValueError("out must have q's dtype")
    else:
        _check_on(out, "out", dev)
    if B == 0:
        return out
    ws_bytes = attention_workspace_bytes(B, Hq, Hkv, D, max_seq_len, q.dtype, n_workgroups,
                                         q.device)
    if ws_bytes > 0 and workspace is None:
        workspace = _cached_workspace(q.device, _stream(q), ws_bytes)
    if ws_bytes > 0:
        _check_on(workspace, "workspace", dev)
        if workspace.numel() * workspace.element_size() < ws_bytes:
            raise ValueError(f"workspace holds {workspace.numel() * workspace.element_size()} "
                             f"bytes, the call needs {ws_bytes}")
    if plan is not None:
        plan.wait_for_build(torch.cuda.current_stream(dev))
    if (key is None) != (value is None):
        raise ValueError("key and value are appended together")
    if key is not None:
        for t, n in ((key, "key"), (value, "value")):
            if t.dim() != 3 or t.shape != (B, Hkv, D) or t.dtype != q.dtype:
                raise ValueError(f"{n} must be [B, Hkv, D] of q's dtype")
            _check_rows(t, n)
            _check_on(t, n, dev)
    ws_ptr = workspace.data_ptr() if (workspace is not None and ws_bytes > 0) else None
    with torch.cuda.device(q.device):
        if key is not None:
            kv = (key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0))
            if plan is not None:
                rc = _lib.load().aegkv_paged_decode_attention_append_planned(
                    out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), *kv,
                    key_cache.data_ptr(), value_cache.data_ptr(), key_cache.stride(0), N,
                    plan.buffer.data_ptr(), plan.nbytes, sl.data_ptr(), B, max_seq_len, Hq, Hkv,
                    D, bs, float(scale), _DTYPES[q.dtype], n_workgroups, ws_ptr,
                    ws_bytes if ws_ptr else 0, _stream(q))
            else:
                rc = _lib.load().aegkv_paged_decode_attention_append(
                    out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), *kv,
                    key_cache.data_ptr(), value_cache.data_ptr(), key_cache.stride(0), N,
                    bt.data_ptr(), bt.size(1), sl.data_ptr(), B, max_seq_len, Hq, Hkv, D, bs,
                    float(scale), _DTYPES[q.dtype], n_workgroups, ws_ptr,
                    ws_bytes if ws_ptr else 0, _stream(q))
        elif plan is not None:
            rc = _lib.load().aegkv_paged_decode_attention_planned(
                out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), key_cache.data_ptr(),
                value_cache.data_ptr(), key_cache.stride(0), N, plan.buffer.data_ptr(),
                plan.nbytes, sl.data_ptr(), B, max_seq_len, Hq, Hkv, D, bs, float(scale),
                _DTYPES[q.dtype], n_workgroups, ws_ptr, ws_bytes if ws_ptr else 0, _stream(q))
        else:
            rc = _lib.load().aegkv_paged_decode_attention(
                out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), key_cache.data_ptr(),
                value_cache.data_ptr(), key_cache.stride(0), N, bt.data_ptr(), bt.size(1),
                sl.data_ptr(), B, max_seq_len, Hq, Hkv, D, bs, float(scale), _DTYPES[q.dtype],
                n_workgroups, ws_ptr, ws_bytes if ws_ptr else 0, _stream(q))
    _lib.check(rc, "paged_decode_attention")
    return out


class _StepPlans:
    """The decode plan of the tables and lengths a caller passes to every
    layer of a step.  vLLM's backend hands each layer's
    flash_attn_with_kvcache the same ``block_table`` and ``cache_seqlens``
    tensors of the step's metadata (worker.py:694-711, :517-523); the plan
    built at the first layer serves the others, whose results are bit-identical
    to unplanned calls.  A cached plan is used only for the very tensor objects
    it was built from (weak references), at the same version counter (an
    in-place torch write bumps it) and data pointer, bound, head count and
    device; anything else builds a new one.  One entry per device: the last
    step's."""

    def __init__(self):
        self._lock = threading.Lock()
        self._by_device: Dict[int, tuple] = {}

    @staticmethod
    def _state(t: torch.Tensor) -> tuple:
        return (t._version, t.data_ptr(), tuple(t.shape), tuple(t.stride()), t.dtype)

    def get(self, block_table: torch.Tensor, cache_seqlens: torch.Tensor, appending: bool,
            max_seq_len: int, n_kv_heads: int):
        """(plan, seq_lens): seq_lens counts the new token when appending;
        plan is None for a batch too large to plan."""
        dev = cache_seqlens.device.index
        key = (self._state(block_table), self._state(cache_seqlens), appending, max_seq_len,
               n_kv_heads)
        with self._lock:
            e = self._by_device.get(dev)
            if e is not None and e[0]() is block_table and e[1]() is cache_seqlens \
                    and e[2] == key:
                return e[3], e[4]
        seq_lens = cache_seqlens.to(torch.int32) + 1 if appending else cache_seqlens
        plan = None
        if 0 < cache_seqlens.numel() <= _PLAN_MAX_BATCH:
            plan = DecodePlan(block_table, seq_lens, max_seq_len, n_kv_heads)
        with self._lock:
            self._by_device[dev] = (weakref.ref(block_table), weakref.ref(cache_seqlens), key,
                                    plan, seq_lens)
        return plan, seq_lens


_PLAN_MAX_BATCH = 2048  # sequences a plan covers (one launch of the kernels)
_step_plans = _StepPlans()


def flash_attn_with_kvcache(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                            k: Optional[torch.Tensor] = None, v: Optional[torch.Tensor] = None,
                            cache_seqlens: Optional[torch.Tensor] = None,
                            block_table: Optional[torch.Tensor] = None,
                            softmax_scale: Optional[float] = None, causal: bool = True,
                            max_seqlen: Optional[int] = None,
                            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """vllm-flash-attn's paged decode call for one query token per sequence:
    ``q [B, 1, Hq, D]`` -> ``[B, 1, Hq, D]``.  With a single query token the
    causal mask admits every cached token, so ``causal`` does not change the
    result.  ``max_seqlen`` (host bound of ``cache_seqlens``) defaults to
    ``block_table.size(1) * block_size``; longer sequences are attended over
    their first ``max_seqlen`` tokens.  With ``k``/``v`` ``[B, 1, Hkv, D]``
    the new token is first written at position ``cache_seqlens[b]`` and the
    attention covers ``cache_seqlens[b] + 1`` tokens (flash-attn's kvcache
    semantics), in one fused call; the bound then grows by the new token.  A
    new token past the table is not written; one past the bound is written but
    not attended, as the separate append and attention would do.  The first
    call with a step's ``block_table``/``cache_seqlens`` tensors builds their
    decode plan, which the step's other layers reuse (same tensor objects and
    versions; see :class:`_StepPlans`)."""
    if q.dim() != 4 or q.size(1) != 1:
        raise NotImplementedError("decode only: q must be [B, 1, Hq, D]")
    if cache_seqlens is None or block_table is None:
        raise ValueError("cache_seqlens and block_table are required (paged cache)")
    B, _, Hq, D = q.shape
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    bs = k_cache.size(1)
    ms = max_seqlen if max_seqlen is not None else block_table.size(1) * bs
    key = value = None
    if k is not None or v is not None:
        if k is None or v is None or k.dim() != 4 or k.size(1) != 1 or v.shape != k.shape:
            raise ValueError("k and v must both be [B, 1, Hkv, D]")
        key, value = k[:, 0], v[:, 0]
        ms = min(ms + 1, block_table.size(1) * bs)
    if not (block_table.is_cuda and cache_seqlens.is_cuda and block_table.dim() == 2
            and block_table.device == q.device and cache_seqlens.device == q.device):
        raise ValueError("block_table and cache_seqlens must be tensors on q's GPU")
    plan, seq_lens = _step_plans.get(block_table, cache_seqlens, key is not None, ms,
                                     k_cache.size(2))
    o = paged_decode_attention(q.view(B, Hq, D), k_cache, v_cache,
                               None if plan else block_table, None if plan else seq_lens,
                               scale, ms, out=None if out is None else out.view(B, Hq, D),
                               plan=plan, key=key, value=value)
    return o.view(B, 1, Hq, D)


def varlen_prefill_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                             cu_seqlens: torch.Tensor, max_seqlen: int, scale: float,
                             causal: bool = True, out: Optional[torch.Tensor] = None
                             ) -> torch.Tensor:
    """Attention of packed sequences: ``q [T, Hq, D]``, ``k, v [T, Hkv, D]``
    (any token stride, dense heads), sequence b = tokens
    ``cu_seqlens[b] .. cu_seqlens[b+1]`` (int32 on the GPU).  Returns
    ``out [T, Hq, D]``.  ``max_seqlen`` is the host bound of the lengths."""
    for x, n in ((q, "q"), (k, "k"), (v, "v")):
        if x.dim() != 3:
            raise ValueError(f"{n} must be [tokens, heads, head_dim]")
        _check_rows(x, n)
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k, v must share a bf16/fp16 dtype")
    T, Hq, D = q.shape
    if k.shape != v.shape or k.size(0) != T or k.size(2) != D:
        raise ValueError("k and v must be [tokens, Hkv, D] with q's tokens and head_dim")
    if cu_seqlens.dtype != torch.int32 or not cu_seqlens.is_cuda or cu_seqlens.dim() != 1 \
            or not cu_seqlens.is_contiguous():
        raise ValueError("cu_seqlens must be a contiguous int32 GPU tensor [batch + 1]")
    for x, n in ((k, "k"), (v, "v"), (cu_seqlens, "cu_seqlens")):
        _check_on(x, n, q.device)
    if out is None:
        out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    elif out.shape != (T, Hq, D) or out.dtype != q.dtype:
        raise ValueError("out must be [tokens, Hq, D] of q's dtype")
    else:
        _check_rows(out, "out")
        _check_on(out, "out", q.device)
    with torch.cuda.device(q.device):
        rc = _lib.load().aegkv_varlen_prefill_attention(
            out.data_ptr(), out.stride(0), q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0),
            v.data_ptr(), v.stride(0), cu_seqlens.data_ptr(), cu_seqlens.numel() - 1,
            int(max_seqlen), T, Hq, k.size(1), D, float(scale), int(bool(causal)),
            _DTYPES[q.dtype], _stream(q))
    _lib.check(rc, "varlen_prefill_attention")
    return out


def flash_attn_varlen_func(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                           max_seqlen_q: int, max_seqlen_k: int, dropout_p: float = 0.0,
                           softmax_scale: Optional[float] = None, causal: bool = False,
                           window_size: Tuple[int, int] = (-1, -1), alibi_slopes=None,
                           deterministic: bool = False, return_attn_probs: bool = False,
                           block_table: Optional[torch.Tensor] = None,
                           out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """vllm-flash-attn's varlen call as the FlashAttention backend makes it for
    a prompt run without cached prefix: the same ``cu_seqlens`` for queries
    and keys.  Dropout, sliding windows, ALiBi, attention probabilities and a
    paged prefix raise NotImplementedError (the reference's models use none)."""
    if dropout_p != 0.0 or tuple(window_size) != (-1, -1) or alibi_slopes is not None \
            or return_attn_probs or block_table is not None:
        raise NotImplementedError("only the plain (causal) prompt run is supported")
    if cu_seqlens_k is not cu_seqlens_q and not torch.equal(cu_seqlens_k, cu_seqlens_q):
        raise NotImplementedError("queries and keys must share cu_seqlens (no cached prefix)")
    if max_seqlen_k != max_seqlen_q:
        raise NotImplementedError("queries and keys must share max_seqlen")
    D = q.size(-1)
    scale = softmax_scale if softmax_scale is not None else 1.0 / math.sqrt(D)
    return varlen_prefill_attention(q, k, v, cu_seqlens_q, max_seqlen_q, scale, causal, out)
