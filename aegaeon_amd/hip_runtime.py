"""The HIP runtime under the method names of the reference's ``CudaRTLibrary``.

The reference's controller reaches the CUDA runtime through
``block_manager.cudart`` (aegaeon/aegaeon/cuda_wrapper.py:43-218, created at
block_manager.py:182 and used at llm.py:386-395): the shared swap file is
page-locked with it and the model cache is handed it.  :class:`HipRTLibrary`
gives the same methods over ``libamdhip64`` (the copy torch has loaded, so one
HIP runtime serves the process): each ``cudaX`` method calls ``hipX`` and
raises ``RuntimeError`` on a non-zero status, as ``CUDART_CHECK`` does;
``cudaEventQuery`` returns a bool.

On the machines this was built on ``hipHostRegister`` of an existing mapping
is refused; :func:`aegaeon_amd.swap_pool.init_cpu_cache` maps the swap file
without it (swaps then go through a pinned bounce buffer), so the controller
does not need ``cudaHostRegister`` for the swap space.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_int, c_size_t, c_uint, c_void_p
from typing import Dict, Optional

HIP_IPC_HANDLE_SIZE = 64  # hip_runtime_api.h


class hipIpcMemHandle_t(ctypes.Structure):
    _fields_ = [("reserved", ctypes.c_byte * HIP_IPC_HANDLE_SIZE)]


class hipIpcEventHandle_t(ctypes.Structure):
    _fields_ = [("reserved", ctypes.c_byte * HIP_IPC_HANDLE_SIZE)]


# HIP name -> (restype, argtypes), for the runtime calls the reference makes
_HIP: Dict[str, tuple] = {
    "hipSetDevice": (c_int, [c_int]),
    "hipDeviceSynchronize": (c_int, []),
    "hipDeviceReset": (c_int, []),
    "hipGetErrorString": (c_char_p, [c_int]),
    "hipMalloc": (c_int, [POINTER(c_void_p), c_size_t]),
    "hipHostRegister": (c_int, [c_void_p, c_size_t, c_uint]),
    "hipFree": (c_int, [c_void_p]),
    "hipMemset": (c_int, [c_void_p, c_int, c_size_t]),
    "hipMemcpy": (c_int, [c_void_p, c_void_p, c_size_t, c_int]),
    "hipIpcGetMemHandle": (c_int, [POINTER(hipIpcMemHandle_t), c_void_p]),
    "hipIpcOpenMemHandle": (c_int, [POINTER(c_void_p), hipIpcMemHandle_t, c_uint]),
    "hipIpcCloseMemHandle": (c_int, [c_void_p]),
    "hipIpcGetEventHandle": (c_int, [POINTER(hipIpcEventHandle_t), c_void_p]),
    "hipIpcOpenEventHandle": (c_int, [POINTER(c_void_p), hipIpcEventHandle_t]),
    "hipStreamWaitEvent": (c_int, [c_void_p, c_void_p, c_uint]),
    "hipEventSynchronize": (c_int, [c_void_p]),
    "hipEventQuery": (c_int, [c_void_p]),
    "hipEventDestroy": (c_int, [c_void_p]),
}

_HIP_MEMCPY_DEFAULT = 4                 # hipMemcpyDefault
_HIP_IPC_MEM_LAZY_ENABLE_PEER_ACCESS = 1

_loaded: Dict[str, Dict[str, object]] = {}


def _functions(so_file: str) -> Dict[str, object]:
    funcs = _loaded.get(so_file)
    if funcs is None:
        import torch  # noqa: F401  (loads torch's libamdhip64 first: one runtime per process)
        lib = ctypes.CDLL(so_file)
        funcs = {}
        for name, (res, args) in _HIP.items():
            f = getattr(lib, name)
            f.restype, f.argtypes = res, args
            funcs[name] = f
        _loaded[so_file] = funcs
    return funcs


class HipRTLibrary:
    """``CudaRTLibrary`` (cuda_wrapper.py:43-218) on the HIP runtime."""

    def __init__(self, so_file: Optional[str] = None):
        self.so_file = so_file or "libamdhip64.so.7"
        self.funcs = _functions(self.so_file)

    def _call(self, name: str, *args) -> None:
        self.CUDART_CHECK(self.funcs[name](*args))

    def CUDART_CHECK(self, result: int) -> None:
        if result != 0:
            raise RuntimeError(f"HIP runtime error: {self.cudaGetErrorString(result)}")

    def cudaGetErrorString(self, error: int) -> str:
        return self.funcs["hipGetErrorString"](error).decode("utf-8")

    def cudaSetDevice(self, device: int) -> None:
        self._call("hipSetDevice", device)

    def cudaDeviceSynchronize(self) -> None:
        self._call("hipDeviceSynchronize")

    def cudaDeviceReset(self) -> None:
        self._call("hipDeviceReset")

    def cudaMalloc(self, size: int) -> c_void_p:
        ptr = c_void_p()
        self._call("hipMalloc", ctypes.byref(ptr), size)
        return ptr

    def cudaHostRegister(self, ptr: c_void_p, size: int) -> None:
        self._call("hipHostRegister", ptr, size, 0)

    def cudaFree(self, devPtr: c_void_p) -> None:
        self._call("hipFree", devPtr)

    def cudaMemset(self, devPtr: c_void_p, value: int, count: int) -> None:
        self._call("hipMemset", devPtr, value, count)

    def cudaMemcpy(self, dst: c_void_p, src: c_void_p, count: int) -> None:
        self._call("hipMemcpy", dst, src, count, _HIP_MEMCPY_DEFAULT)

    def cudaIpcGetMemHandle(self, devPtr: c_void_p) -> hipIpcMemHandle_t:
        handle = hipIpcMemHandle_t()
        self._call("hipIpcGetMemHandle", ctypes.byref(handle), devPtr)
        return handle

    def cudaIpcOpenMemHandle(self, handle: hipIpcMemHandle_t) -> c_void_p:
        ptr = c_void_p()
        self._call("hipIpcOpenMemHandle", ctypes.byref(ptr), handle,
                   _HIP_IPC_MEM_LAZY_ENABLE_PEER_ACCESS)
        return ptr

    def cudaIpcCloseMemHandle(self, devPtr: c_void_p) -> None:
        self._call("hipIpcCloseMemHandle", devPtr)

    def cudaIpcGetEventHandle(self, event: c_void_p) -> hipIpcEventHandle_t:
        handle = hipIpcEventHandle_t()
        self._call("hipIpcGetEventHandle", ctypes.byref(handle), event)
        return handle

    def cudaIpcOpenEventHandle(self, handle: hipIpcEventHandle_t) -> c_void_p:
        event = c_void_p()
        self._call("hipIpcOpenEventHandle", ctypes.byref(event), handle)
        return event

    def cudaStreamWaitEvent(self, stream: c_void_p, event: c_void_p, flags: int = 0) -> None:
        self._call("hipStreamWaitEvent", stream, event, flags)

    def cudaEventSynchronize(self, event: c_void_p) -> None:
        self._call("hipEventSynchronize", event)

    def cudaEventQuery(self, event: c_void_p) -> bool:
        return self.funcs["hipEventQuery"](event) == 0

    def cudaEventDestroy(self, event: c_void_p) -> None:
        self._call("hipEventDestroy", event)
