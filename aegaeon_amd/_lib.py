"""ctypes binding of ``libaegkv.so`` (the C ABI declared in include/aegkv.h).

The library is built in-tree by ``aegaeon_amd.csrc.build``.  Loading fails
loudly when it is missing: there is no CPU fallback for any op of the path.
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_float, c_int, c_int32, c_int64, c_uint64, c_void_p
from pathlib import Path
from typing import Dict, Optional

LIB_PATH = Path(__file__).resolve().with_name("libaegkv.so")
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "aegkv.h"

AEGKV_DTYPE_BF16 = 0
AEGKV_DTYPE_FP16 = 1

_i64p = POINTER(c_int64)
_i32p = POINTER(c_int32)

# name -> (restype, argtypes); mirrors include/aegkv.h
SIGNATURES: Dict[str, tuple] = {
    "aegkv_strerror": (c_char_p, [c_int]),
    "aegkv_version": (c_int, []),
    "aegkv_init": (c_int, []),
    "aegkv_swap_blocks": (c_int, [_i64p, _i64p, c_int64, c_int, c_void_p, c_uint64, c_void_p,
                                  c_uint64, c_uint64, c_void_p, c_uint64, c_void_p]),
    "aegkv_swap_blocks_bounced": (c_int, [_i64p, _i64p, c_int64, c_int, c_void_p, c_uint64,
                                          c_void_p, c_uint64, c_uint64, c_void_p, c_uint64,
                                          c_void_p, c_uint64, c_void_p]),
    "aegkv_signals_create": (c_int, [c_int64, POINTER(c_void_p), c_void_p]),
    "aegkv_signals_destroy": (c_int, [c_void_p]),
    "aegkv_signals_open": (c_int, [c_void_p, POINTER(c_void_p), POINTER(c_int64)]),
    "aegkv_signals_close": (c_int, [c_void_p]),
    "aegkv_signal_set": (c_int, [c_void_p, c_uint64, c_void_p]),
    "aegkv_signal_wait": (c_int, [c_void_p, c_uint64, c_uint64, c_void_p, c_void_p]),
    "aegkv_signal_read": (c_int, [c_void_p, POINTER(c_uint64), c_void_p]),
    "aegkv_copy_blocks": (c_int, [c_void_p, c_uint64, c_void_p, c_uint64, _i64p, _i64p, c_int64,
                                  c_uint64, c_void_p]),
    "aegkv_pack_blocks": (c_int, [c_void_p, c_uint64, _i64p, c_int64, c_void_p, c_uint64,
                                  c_void_p]),
    "aegkv_scatter_blocks": (c_int, [c_void_p, _i64p, c_int64, c_void_p, c_uint64, c_uint64,
                                     c_void_p]),
    "aegkv_defrag_blocks": (c_int, [c_void_p, c_uint64, _i64p, _i64p, c_int64, c_uint64,
                                    c_void_p]),
    "aegkv_kv_append": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_void_p,
                                c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int32,
                                c_int32, c_int32, c_int32, c_int32, c_void_p]),
    "aegkv_gather_tokens": (c_int, [c_void_p, c_void_p, c_int64, c_int64, c_int64, c_void_p,
                                    c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
                                    c_void_p, c_int64, c_int64, c_int32, c_int32, c_int32,
                                    c_int32, c_int32, c_void_p]),
    "aegkv_paged_decode_attention_workspace_size": (c_int64, [c_int32, c_int32, c_int32, c_int32,
                                                              c_int32, c_int32, c_int32]),
    "aegkv_prepare_inputs": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int32,
                                     c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "aegkv_paged_decode_attention": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                             c_void_p, c_int64, c_int64, c_void_p, c_int32,
                                             c_void_p, c_int32, c_int32, c_int32, c_int32,
                                             c_int32, c_int32, c_float, c_int32, c_int32,
                                             c_void_p, c_uint64, c_void_p]),
    "aegkv_paged_decode_attention_noalloc": (c_int, [c_void_p, c_int64, c_void_p, c_int64,
                                                     c_void_p, c_void_p, c_int64, c_int64,
                                                     c_void_p, c_int32, c_void_p, c_int32,
                                                     c_int32, c_int32, c_int32, c_int32,
                                                     c_int32, c_float, c_int32, c_int32,
                                                     c_void_p]),
    "aegkv_paged_decode_attention_append": (c_int, [c_void_p, c_int64, c_void_p, c_int64,
                                                    c_void_p, c_int64, c_void_p, c_int64,
                                                    c_void_p, c_void_p, c_int64, c_int64,
                                                    c_void_p, c_int32, c_void_p, c_int32,
                                                    c_int32, c_int32, c_int32, c_int32,
                                                    c_int32, c_float, c_int32, c_int32,
                                                    c_void_p, c_uint64, c_void_p]),
    "aegkv_paged_decode_attention_append_planned": (c_int, [c_void_p, c_int64, c_void_p,
                                                            c_int64, c_void_p, c_int64,
                                                            c_void_p, c_int64, c_void_p,
                                                            c_void_p, c_int64, c_int64,
                                                            c_void_p, c_uint64, c_void_p,
                                                            c_int32, c_int32, c_int32, c_int32,
                                                            c_int32, c_int32, c_float, c_int32,
                                                            c_int32, c_void_p, c_uint64,
                                                            c_void_p]),
    "aegkv_paged_decode_plan_size": (c_int64, [c_int32, c_int32, c_int32, c_int32]),
    "aegkv_paged_decode_plan": (c_int, [c_void_p, c_int32, c_void_p, c_int32, c_int32, c_int32,
                                        c_int32, c_void_p, c_uint64, c_void_p]),
    "aegkv_paged_decode_attention_planned": (c_int, [c_void_p, c_int64, c_void_p, c_int64,
                                                     c_void_p, c_void_p, c_int64, c_int64,
                                                     c_void_p, c_uint64, c_void_p, c_int32,
                                                     c_int32, c_int32, c_int32, c_int32,
                                                     c_int32, c_float, c_int32, c_int32,
                                                     c_void_p, c_uint64, c_void_p]),
    "aegkv_varlen_prefill_attention": (c_int, [c_void_p, c_int64, c_void_p, c_int64, c_void_p,
                                               c_int64, c_void_p, c_int64, c_void_p, c_int32,
                                               c_int32, c_int64, c_int32, c_int32, c_int32,
                                               c_float, c_int32, c_int32, c_void_p]),
    # block manager (host bookkeeping)
    "aegkv_bm_create": (c_int, [c_int64, c_int64, POINTER(c_void_p)]),
    "aegkv_bm_destroy": (None, [c_void_p]),
    "aegkv_bm_set_wait": (c_int, [c_void_p, c_void_p, c_void_p]),
    "aegkv_bm_define_shape": (c_int, [c_void_p, c_int32, c_uint64]),
    "aegkv_bm_register_gpu_space": (c_int, [c_void_p, c_int32, c_int64, c_int32]),
    "aegkv_bm_allocate": (c_int, [c_void_p, c_int32, c_void_p, c_void_p, c_int64]),
    "aegkv_bm_free": (c_int, [c_void_p, c_int64]),
    "aegkv_bm_move": (c_int, [c_void_p, c_void_p, c_int64, c_int32, _i64p, _i64p, _i32p, _i32p]),
    "aegkv_bm_move_ids": (c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
                                  _i64p]),
    "aegkv_bm_complete_moves": (c_int, [c_void_p, c_int32, c_int32, c_int64]),
    "aegkv_bm_pending": (c_int, [c_void_p, _i64p, _i32p, _i32p, _i64p]),
    "aegkv_bm_resume": (c_int, [c_void_p, c_int64, _i64p, _i64p, _i32p, _i32p]),
    "aegkv_bm_cancel": (c_int, [c_void_p, c_int64]),
    "aegkv_bm_complete_move": (c_int, [c_void_p, c_int32, c_int32, c_int64]),
    "aegkv_bm_reclaim_slabs": (c_int, [c_void_p]),
    "aegkv_bm_table": (c_int, [c_void_p, c_int64, _i32p, _i32p, _i64p, c_void_p, c_int64]),
    "aegkv_bm_flat_tables": (c_int, [c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64]),
    "aegkv_bm_stats": (c_int, [c_void_p, c_int32, c_int32, _i64p, _i64p, _i64p, _i64p]),
    "aegkv_bm_free_list": (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_int64, _i64p]),
}

# int (*)(void* ctx, int32_t location, int32_t shape, int64_t serial)
BM_WAIT_FN = ctypes.CFUNCTYPE(c_int, c_void_p, c_int32, c_int32, c_int64)


class AegkvError(RuntimeError):
    """A non-zero status from the C ABI (message from aegkv_strerror)."""

    def __init__(self, code: int, message: str, op: str = ""):
        super().__init__(f"{op}: {message} (status {code})" if op else f"{message} (status {code})")
        self.code = code


_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def load(path: Optional[Path] = None) -> ctypes.CDLL:
    """Load (once) and type the library.  Raises if it has not been built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise RuntimeError(
                f"{p} is missing: build the HIP KV data path first "
                "(python -m aegaeon_amd.csrc.build)")
        lib = ctypes.CDLL(str(p))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if path is None:
            _lib = lib
        return lib


def strerror(code: int) -> str:
    return load().aegkv_strerror(code).decode()


def check(code: int, op: str = "") -> None:
    if code != 0:
        raise AegkvError(code, strerror(code), op)


def declared_symbols(header: Path = HEADER_PATH) -> list:
    """Function names declared in include/aegkv.h."""
    import re
    text = header.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(aegkv_\w+)\s*\(", text, re.M)))
