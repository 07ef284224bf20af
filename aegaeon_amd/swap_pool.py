"""The node-wide CPU swap space as a shared file, and move events shared
between processes.

The reference keeps every worker's CPU swap space in one file,
``/dev/shm/aegaeon_cpu_cache`` (aegaeon/aegaeon/llm.py:36,297-318), of
``cpu_num_slabs * cpu_slab_size_bytes`` bytes mapped shared as float16 by the
controller and by every worker (worker.py:130-147), so that a request swapped
out by one engine's worker can be swapped in by another's.  Block ``b`` of a
shape with ``bb`` bytes per block lives at byte ``b * bb`` of the file (the
slab arithmetic of block_manager.py:186-199,242-245).  :func:`init_cpu_cache`
maps the same file the same way.

The reference page-locks the mapping with ``cudaHostRegister`` so that the
swap kernel can DMA into it.  Where registering an existing mapping is not
available (``hipHostRegister`` is refused on the machines this was built on),
the mapping stays pageable and :func:`aegaeon_amd.ops.swap` reaches it through
a pinned bounce buffer (``bounce=``, aegkv_swap_blocks_bounced); the file's
layout and contents are the same either way.

Move events cross processes where the reference exports interprocess CUDA
events (``reduce_cuda_event`` / ``rebuild_cuda_event``, utils.py:306-331).
The HIP runtime these kernels run on creates such events but refuses to
record them (``hipEventRecord`` returns invalid argument for an event created
with ``hipEventInterprocess``), so a move is signalled through
:class:`SignalArray` instead: timeline words in device memory shared with
``hipIpcGetMemHandle``, set by a one-lane kernel behind the move on the
producer's stream and awaited by a one-lane kernel on the consumer's stream
(aegkv_signal_set / aegkv_signal_wait).  An exported move is
:data:`EventHandle` ``(device, pid, array handle, word, serial)``; the pid
tells a process its own handles apart (the reference uses the device alone,
one worker process per GPU), and a process never opens its own array.
"""
from __future__ import annotations

import ctypes
import os
from typing import Dict, Optional, Tuple

import torch

from . import _lib

AEGAEON_CPU_CACHE_FILENAME = "/dev/shm/aegaeon_cpu_cache"  # llm.py:36

# (device, exporting pid, signal-array IPC handle, word, serial)
EventHandle = Tuple[int, int, bytes, int, int]


def init_cpu_cache(cpu_num_slabs: int, cpu_slab_size_bytes: int,
                   filename: str = AEGAEON_CPU_CACHE_FILENAME) -> torch.Tensor:
    """The shared swap space (``Controller._init_cpu_cache``, llm.py:297-318;
    ``Worker.__init__``, worker.py:130-142): the file is created (zero-filled,
    sparse) when missing and mapped shared as ``cpu_num_slabs *
    cpu_slab_size_bytes // 2`` float16 elements.  Every process that calls this
    with the same arguments sees the same bytes."""
    size = cpu_num_slabs * cpu_slab_size_bytes
    if size <= 0 or size % 2:
        raise ValueError("the swap space must hold a positive, even number of bytes")
    return torch.from_file(filename, shared=True, size=size // 2, dtype=torch.float16)


def bounce_buffer(nbytes: int) -> torch.Tensor:
    """A pinned host buffer for :func:`aegaeon_amd.ops.swap`'s ``bounce=``.  A
    swap uses it as two halves (one chunk's host copy overlaps the next chunk's
    DMA) and moves min(staging, half the bounce buffer) bytes per chunk."""
    return torch.empty(nbytes, dtype=torch.uint8, pin_memory=True)


class SignalArray:
    """Timeline words in device memory that other processes can open: the
    creator's words come from aegkv_signals_create, an opened array from
    aegkv_signals_open on the creator's 64-byte handle (which also gives the
    word count, so every process checks its word indexes)."""

    def __init__(self, n_words: int = 64, device=None):
        self._lib = _lib.load()
        self.device = torch.device("cuda", torch.cuda.current_device()) if device is None \
            else torch.device(device)
        self.n_words = int(n_words)
        ptr, handle = ctypes.c_void_p(), (ctypes.c_char * 64)()
        with torch.cuda.device(self.device):
            _lib.check(self._lib.aegkv_signals_create(self.n_words, ctypes.byref(ptr), handle),
                       "signals_create")
        self.ptr, self.handle, self.owned = ptr.value, bytes(handle), True
        self._read_stream = None
        _created[self.handle] = self

    @classmethod
    def open(cls, handle: bytes, device) -> "SignalArray":
        self = cls.__new__(cls)
        self._lib = _lib.load()
        self.device = torch.device(device)
        if len(handle) != 64:
            raise ValueError("a signal-array handle is 64 bytes")
        ptr, n = ctypes.c_void_p(), ctypes.c_int64()
        with torch.cuda.device(self.device):
            _lib.check(self._lib.aegkv_signals_open(bytes(handle), ctypes.byref(ptr),
                                                    ctypes.byref(n)), "signals_open")
        self.ptr, self.handle, self.owned = ptr.value, bytes(handle), False
        self.n_words = int(n.value)
        self._read_stream = None
        return self

    def word(self, i: int) -> int:
        i = int(i)
        if not 0 <= i < self.n_words:
            raise IndexError(f"signal word {i} outside the array's {self.n_words}")
        if not self.ptr:
            raise ValueError("the signal array is closed")
        return self.ptr + 8 * i

    def signal(self, stream: torch.cuda.Stream, i: int, value: int) -> None:
        """After ``stream``'s earlier work, word ``i`` = ``value``."""
        _lib.check(self._lib.aegkv_signal_set(self.word(i), int(value), stream.cuda_stream),
                   "signal_set")

    def read(self, i: int) -> int:
        """The current value of word ``i``, read from the host (a copy on a
        stream of this array's own, so no other work is waited for)."""
        word = self.word(i)
        if self._read_stream is None:
            self._read_stream = torch.cuda.Stream(device=self.device)
        value = ctypes.c_uint64()
        with torch.cuda.device(self.device):
            _lib.check(self._lib.aegkv_signal_read(word, ctypes.byref(value),
                                                   self._read_stream.cuda_stream), "signal_read")
        return int(value.value)

    def wait(self, stream: torch.cuda.Stream, i: int, value: int, timed_out: torch.Tensor,
             timeout_s: float = 120.0) -> None:
        """``stream``'s later work waits until word ``i`` >= ``value`` (or the
        timeout, which sets the int32 word ``timed_out``: pinned host memory,
        which the host reads without synchronising, or a word on the stream's
        GPU)."""
        on_gpu = timed_out.is_cuda and timed_out.device == stream.device
        if not ((on_gpu or (not timed_out.is_cuda and timed_out.is_pinned()))
                and timed_out.dtype == torch.int32 and timed_out.numel() >= 1):
            raise ValueError("timed_out must be an int32 tensor in pinned host memory or on "
                             "the stream's GPU")
        _lib.check(self._lib.aegkv_signal_wait(self.word(i), int(value),
                                               max(1, int(timeout_s * 1e6)),
                                               timed_out.data_ptr(), stream.cuda_stream),
                   "signal_wait")

    def close(self) -> None:
        """Free (creator) or unmap (opener) the words once every kernel this
        process enqueued on them has ended (the device is synchronised)."""
        if self.ptr:
            with torch.cuda.device(self.device):
                torch.cuda.synchronize(self.device)
                rc = (self._lib.aegkv_signals_destroy if self.owned
                      else self._lib.aegkv_signals_close)(self.ptr)
            self.ptr = 0
            _created.pop(self.handle, None)
            _lib.check(rc, "signals_close")


def reduce_event(array: SignalArray, word: int, serial: int) -> EventHandle:
    """utils.py:306-315: the handle of the move that sets ``word`` of this
    process's ``array`` to ``serial``."""
    array.word(word)  # bounds check
    return (array.device.index, os.getpid(), array.handle, int(word), int(serial))


_opened: Dict[bytes, SignalArray] = {}
_created: Dict[bytes, SignalArray] = {}   # this process's own arrays, by handle


def rebuild_event(handle: EventHandle) -> Optional[Tuple[SignalArray, int, int]]:
    """utils.py:318-331: ``(array, word, serial)`` to wait on, opening the
    exporter's array once per process.  A handle this process exported is
    served by its own array (a process never opens its own); None when that
    array has been closed."""
    device, pid, raw, word, serial = handle
    if pid == os.getpid():
        arr = _created.get(bytes(raw))
        return None if arr is None else (arr, int(word), int(serial))
    arr = _opened.get(raw)
    if arr is None:
        arr = _opened[raw] = SignalArray.open(raw, torch.device("cuda", device))
    return arr, int(word), int(serial)


def query_event(handle: EventHandle) -> bool:
    """Whether the move behind ``handle`` has finished (the host-side
    ``cudaEventQuery`` of a rebuilt event, block_manager.py:387-398)."""
    opened = rebuild_event(handle)
    if opened is None:
        raise ValueError("the signal array of this move handle was closed")
    arr, word, serial = opened
    return arr.read(word) >= serial


def close_opened() -> None:
    """Close every signal array this process opened (once nothing enqueued
    still waits on them)."""
    while _opened:
        _, arr = _opened.popitem()
        arr.close()

