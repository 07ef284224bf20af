"""The worker's side of a KV move: streams, move events and the swap call.

:class:`KVSwapWorker` keeps the stream and event protocol of the reference's
``Worker`` (aegaeon/aegaeon/worker.py:130-158, 716-839) for one GPU:

* a swap-in and a swap-out stream (both at the default priority), so the two
  directions run concurrently with each other and with the compute stream;
* :meth:`swap_blocks` waits on the requests' previous move events, enqueues
  :func:`aegaeon_amd.ops.swap` on the direction's stream, records a new event
  after it and files that event under every moved request
  (``move_event_table``, worker.py:752-815);
* :meth:`ready_mask` / :meth:`wait_for_moves` are the compute side: a request
  whose last move event has not completed is not ready; when no request of a
  batch is ready, the compute stream waits on the last event of each
  (worker.py:473-500).

The block manager (:class:`aegaeon_amd.block_manager.BlockManager`) calls
:meth:`swap_blocks` through its per-engine remote callable with the id lists
of ``move_requests`` and keeps the returned event as the move's handle; the
manager's reclaim waits on it before the source blocks are handed out again
(block_manager.py:360-408).

One departure, by design: the reference synchronises the compute stream
after every forward (worker.py:524), which orders a later swap-out after the
forward's K/V writes.  Here that order is explicit: a swap waits on the
events passed as ``after`` (for example one recorded on the compute stream
after the step's append), so the compute stream need not be synchronised.

With ``interprocess=True`` every move also sets a word of the worker's
:class:`aegaeon_amd.swap_pool.SignalArray` (one word per swap stream, the
move's serial), :meth:`export` gives the handle another process waits on
(the reference's ``reduce_cuda_event``, utils.py:306-315), and a source entry
may be such a handle: :meth:`swap_blocks` then makes its stream wait on that
word (``rebuild_cuda_event``, utils.py:318-331; worker.py:795-812), from this
process's own array when it exported the handle, so the wait needs no request
id.  A wait that times out sets :attr:`timed_out`, a word of pinned host
memory; the host checks it without synchronising at every point where it
treats moves as complete (:meth:`ready_mask`, :meth:`wait_for_moves`,
:meth:`wait_for_all_move_in` / ``_out``) and raises ``TimeoutError`` there,
since the work behind the wait ran unordered.  A pageable swap space (the shared file of
:func:`aegaeon_amd.swap_pool.init_cpu_cache` where it cannot be page-locked)
is reached through pinned bounce buffers the worker owns.
"""
from __future__ import annotations

from collections import defaultdict
from typing import Dict, Iterable, List, Optional, Sequence, Union

import torch

from . import ops, swap_pool

EventLike = Union[torch.cuda.Event, swap_pool.EventHandle, Sequence, None]


def _is_handle(x) -> bool:
    return isinstance(x, tuple) and len(x) == 5 and isinstance(x[2], (bytes, bytearray))


def _events(x: EventLike) -> List:
    """Flatten events and exported handles (kept as they are)."""
    if x is None:
        return []
    if isinstance(x, torch.cuda.Event) or _is_handle(x):
        return [x]
    out: List = []
    for e in x:
        out.extend(_events(e))
    return out


class KVSwapWorker:
    """Swap streams and move events of one GPU's KV cache (worker.py:130-158).

    ``kv_cache``: the GPU storage ``[N, L, 2, 16, Hkv, D]``; ``kv_swap``: the
    pinned CPU swap space with the same block size; ``compute_stream``: the
    stream the forward runs on (default: the current stream)."""

    def __init__(self, kv_cache: torch.Tensor, kv_swap: torch.Tensor,
                 compute_stream: Optional[torch.cuda.Stream] = None,
                 interprocess: bool = False, bounce_bytes: int = 256 << 20,
                 wait_timeout_s: float = 120.0):
        if not kv_cache.is_cuda:
            raise ValueError("kv_cache must be a GPU tensor")
        self.device = kv_cache.device
        self.kv_cache = kv_cache
        self.kv_swap = kv_swap
        self.interprocess = interprocess
        self.signals = swap_pool.SignalArray(2, self.device) if interprocess else None
        self._serial = {True: 0, False: 0}       # per swap stream (word 1: swap-in)
        self.timed_out = torch.zeros(1, dtype=torch.int32, pin_memory=True)
        self.wait_timeout_s = wait_timeout_s  # bound of a wait on a cross-process move
        # one bounce buffer per direction: the two swap streams run concurrently
        self.bounce = None if kv_swap.is_pinned() else {
            d: swap_pool.bounce_buffer(bounce_bytes) for d in (True, False)}
        self.swap_in_stream = torch.cuda.Stream(device=self.device)
        self.swap_out_stream = torch.cuda.Stream(device=self.device)
        self.compute_stream = compute_stream or torch.cuda.current_stream(self.device)
        # request id -> events of its moves, oldest first (worker.py:158)
        self.move_event_table: Dict[int, List[torch.cuda.Event]] = defaultdict(list)

    # -- the swap (worker.py:716-770) -------------------------------------------
    def swap_blocks(self, request_ids: Sequence[int], source_block_ids: Sequence[int],
                    target_block_ids: Sequence[int], source_events: Iterable[EventLike],
                    is_swap_in: bool, after: EventLike = None) -> torch.cuda.Event:
        """Copy ``source_block_ids[i]`` to ``target_block_ids[i]`` (CPU->GPU when
        ``is_swap_in``) on the direction's stream, after the requests' previous
        moves (``source_events``, one entry per request: None, an event, or a
        list) and the events in ``after``; returns the event recorded behind
        the copy, also filed under every request."""
        stream = self.swap_in_stream if is_swap_in else self.swap_out_stream
        new_event = torch.cuda.Event()
        self._wait_source_events(stream, request_ids, source_events)
        for e in _events(after):
            self._wait(stream, e)
        with torch.cuda.stream(stream):
            ops.swap(source_block_ids, target_block_ids, is_swap_in, self.kv_cache,
                     self.kv_swap, bounce=None if self.bounce is None else self.bounce[is_swap_in])
        new_event.record(stream)
        # filed only once recorded: a swap that raised leaves every request's
        # last event as it was
        for rid in request_ids:
            self.move_event_table[rid].append(new_event)
        if self.signals is not None:
            word = 1 if is_swap_in else 0
            self._serial[is_swap_in] += 1
            self.signals.signal(stream, word, self._serial[is_swap_in])
            new_event.aegkv_signal = (word, self._serial[is_swap_in])
        return new_event

    def export(self, event: torch.cuda.Event) -> swap_pool.EventHandle:
        """The handle of a move of this worker that another process waits on
        (``reduce_cuda_event``); needs ``interprocess=True``."""
        if self.signals is None or not hasattr(event, "aegkv_signal"):
            raise ValueError("only moves of an interprocess worker can be exported")
        return swap_pool.reduce_event(self.signals, *event.aegkv_signal)

    def check_timeouts(self) -> None:
        """Raise if a wait on a cross-process move gave up (a host read of a
        pinned word: no synchronisation; it reports waits that have ended)."""
        if int(self.timed_out[0]):
            raise TimeoutError("a wait on another process's move timed out; the work behind it "
                               "ran unordered")

    def _wait(self, stream: torch.cuda.Stream, e) -> None:
        if _is_handle(e):
            opened = swap_pool.rebuild_event(e)
            if opened is None:
                raise ValueError("the signal array of this move handle was closed")
            arr, word, serial = opened
            arr.wait(stream, word, serial, self.timed_out, self.wait_timeout_s)
            return
        stream.wait_event(e)

    def _wait_source_events(self, stream: torch.cuda.Stream, request_ids: Sequence[int],
                            source_events: Iterable[EventLike]) -> None:
        """worker.py:772-815: a request with a move in flight is waited on
        before anything else touches its blocks; the request's own last event
        stands in when its entry holds no event."""
        source_events = list(source_events)
        if len(source_events) != len(request_ids):
            raise ValueError("one source event entry per request")
        for rid, handles in zip(request_ids, source_events):
            if handles is not None:
                evs = _events(handles)
                if not evs and self.move_event_table.get(rid):
                    evs = [self.move_event_table[rid][-1]]
                for e in evs:
                    self._wait(stream, e)

    # -- the compute side (worker.py:473-500) -------------------------------------
    def ready_mask(self, request_ids: Sequence[int]) -> List[bool]:
        """A request is ready when it has no move event or its last one has
        completed (a non-blocking query)."""
        self.check_timeouts()
        mask = []
        for rid in request_ids:
            evs = self.move_event_table.get(rid)
            mask.append(not evs or evs[-1].query())
        return mask

    def wait_for_moves(self, request_ids: Sequence[int],
                       stream: Optional[torch.cuda.Stream] = None) -> List[bool]:
        """The forward's gate: returns the ready mask; when no request is
        ready, ``stream`` (default: the compute stream) waits on the last
        move event of every request and all of them count as ready."""
        mask = self.ready_mask(request_ids)
        if request_ids and not any(mask):
            s = stream or self.compute_stream
            for rid in request_ids:
                evs = self.move_event_table.get(rid)
                if evs:
                    s.wait_event(evs[-1])
            mask = [True] * len(request_ids)
        return mask

    # -- bookkeeping (worker.py:817-839) ------------------------------------------
    def clear_request_resource(self, request_id: int) -> None:
        self.move_event_table.pop(request_id, None)

    def clear_request_resource_batched(self, request_ids: Sequence[int]) -> None:
        for rid in request_ids:
            self.clear_request_resource(rid)

    def wait_for_all_move_in(self) -> None:
        self.swap_in_stream.synchronize()
        self.check_timeouts()

    def wait_for_all_move_out(self) -> None:
        self.swap_out_stream.synchronize()
        self.check_timeouts()

    def remote_callable(self, after: EventLike = None):
        """The block manager's per-engine callable: ``remote("swap_blocks",
        request_ids, src, dst, source_handles, is_swap_in)`` (block_manager.py:
        833-848) runs :meth:`swap_blocks` and returns its event as the move's
        handle; ``remote("clear_request_resource_batched", request_ids)``
        (block_manager.py:770-776) drops freed requests' events.  ``after`` is
        evaluated per swap when it is a callable returning events."""
        def remote(method, *args):
            if method == "swap_blocks":
                request_ids, src, dst, source_handles, is_swap_in = args
                extra = after() if callable(after) else after
                return self.swap_blocks(request_ids, src, dst, source_handles, is_swap_in,
                                        after=extra)
            if method == "clear_request_resource_batched":
                (request_ids,) = args
                return self.clear_request_resource_batched(request_ids)
            raise ValueError(f"unknown worker method {method!r}")
        return remote
