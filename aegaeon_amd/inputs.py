"""Per-step model inputs built on the GPU, with the reference's outputs.

:func:`prepare_model_inputs` takes what ``Worker._prepare_model_inputs``
(aegaeon/aegaeon/worker.py:554-713) takes — the batch's ``RequestMeta`` tuples
``(request_id, tokens, seq_len, context_len)`` (aegaeon/aegaeon/request.py:
96-102), sorted prefill -> decode, and their block tables — and returns the
same ``(input_tokens, input_positions, metadata)``, where ``metadata`` holds the
keyword arguments the reference passes to the attention backend's
``make_metadata`` (worker.py:694-711).  The per-token slot-mapping loop
(worker.py:628-633), the 0-padded table build (utils.py:241-257) and the eight
host-to-device tensors become one upload and one gfx950 kernel
(``aegkv_prepare_inputs``).
"""
from __future__ import annotations

from typing import Dict, List, Sequence, Tuple

import numpy as np
import torch

from . import _lib

try:
    from . import _listpack
except ImportError as e:  # built beside libaegkv.so by csrc/build.py
    raise ImportError("aegaeon_amd._listpack is not built: run __graft_entry__.build() "
                      "(aegaeon_amd/csrc/build.py)") from e

BLOCK_SIZE = 16  # aegaeon/aegaeon/config.py:13


def _ptr(a: np.ndarray):
    return a.ctypes.data if a.size else None


def prepare_model_inputs(requests: Sequence[Tuple], block_tables: Sequence[Sequence[int]],
                         device, block_size: int = BLOCK_SIZE
                         ) -> Tuple[torch.Tensor, torch.Tensor, Dict]:
    """GPU form of ``Worker._prepare_model_inputs``.

    Returns ``(input_tokens int64 [T], input_positions int64 [T], metadata)``
    with ``metadata`` = ``num_prefills, slot_mapping (int64 [T]),
    num_prefill_tokens, num_decode_tokens, seq_lens (list), seq_lens_tensor
    (int32), max_query_len, max_prefill_seq_len, max_decode_seq_len,
    query_start_loc (int32 [B+1]), seq_start_loc (int32 [B+1]),
    context_lens_tensor (int32), block_tables (int32 [B, max table len]),
    use_cuda_graph=False``.  Raises ``AegkvError`` for a table that does not
    cover its sequence, like the reference's index error.
    """
    if len(requests) == 0:
        raise ValueError("empty batch")  # the reference asserts (worker.py:594)
    if len(block_tables) != len(requests):
        raise ValueError("one block table per request")
    # the lists read through the CPython API in one pass each (the block
    # manager's tables, the requests' lengths and new tokens)
    ids, offsets = _listpack.pack_tables(block_tables)
    seq, ctx, tokens = _listpack.pack_requests(requests)
    return prepare_inputs_from_arrays(np.frombuffer(ids, dtype=np.int32),
                                      np.frombuffer(offsets, dtype=np.int64),
                                      np.frombuffer(seq, dtype=np.int32),
                                      np.frombuffer(ctx, dtype=np.int32),
                                      np.frombuffer(tokens, dtype=np.int64), device, block_size)


def prepare_inputs_from_arrays(table_ids: np.ndarray, table_offsets: np.ndarray,
                               seq_lens: np.ndarray, context_lens: np.ndarray,
                               tokens: np.ndarray, device, block_size: int = BLOCK_SIZE
                               ) -> Tuple[torch.Tensor, torch.Tensor, Dict]:
    """The same outputs as :func:`prepare_model_inputs`, from arrays: request
    b's block table is ``table_ids[table_offsets[b]:table_offsets[b + 1]]``
    (int32; the layout ``BlockManager.flat_block_tables`` returns), its
    lengths ``seq_lens[b]`` / ``context_lens[b]`` (int32) and its new tokens
    the next ``seq_len - context_len`` entries of ``tokens`` (int64)."""
    device = torch.device(device)
    ids = np.ascontiguousarray(table_ids, dtype=np.int32)
    offsets = np.ascontiguousarray(table_offsets, dtype=np.int64)
    seq = np.ascontiguousarray(seq_lens, dtype=np.int32)
    ctx = np.ascontiguousarray(context_lens, dtype=np.int32)
    tokens = np.ascontiguousarray(tokens, dtype=np.int64)
    B = seq.size
    if B == 0:
        raise ValueError("empty batch")  # the reference asserts (worker.py:594)
    if ctx.size != B or offsets.size != B + 1:
        raise ValueError("one context length and one table per request")
    qlen = seq.astype(np.int64) - ctx
    is_prompt = ctx == 0
    lens = np.diff(offsets)
    # decode rows keep their table, prefill rows are empty (worker.py:600-605)
    pad_width = int(lens[~is_prompt].max()) if (~is_prompt).any() else 0
    T = int(qlen.sum())
    if tokens.size != T:
        raise ValueError("tokens must hold every request's new tokens")

    # the outputs are views of one int32 and one int64 allocation (two
    # allocator calls per step instead of eight)
    w32 = torch.empty(B * pad_width + 4 * B + 2, dtype=torch.int32, device=device)
    w64 = torch.empty(3 * T, dtype=torch.int64, device=device)
    bt_out = w32[:B * pad_width].view(B, pad_width)
    seq_t, ctx_t, qsl, ssl = torch.split(w32[B * pad_width:], [B, B, B + 1, B + 1])
    slots, positions, toks = torch.split(w64, [T, T, T])
    with torch.cuda.device(device):
        rc = _lib.load().aegkv_prepare_inputs(
            _ptr(ids), offsets.ctypes.data, seq.ctypes.data, ctx.ctypes.data, _ptr(tokens), B,
            block_size, pad_width, bt_out.data_ptr() if pad_width else None,
            slots.data_ptr() if T else None, positions.data_ptr() if T else None,
            toks.data_ptr() if T else None, seq_t.data_ptr(), ctx_t.data_ptr(), qsl.data_ptr(),
            ssl.data_ptr(), T, torch.cuda.current_stream(device).cuda_stream)
    _lib.check(rc, "prepare_model_inputs")
    prefill_lens = seq[is_prompt]
    decode_lens = seq[~is_prompt]
    metadata = dict(
        num_prefills=int(is_prompt.sum()),
        slot_mapping=slots,
        num_prefill_tokens=int(qlen[is_prompt].sum()),
        num_decode_tokens=int(qlen[~is_prompt].sum()),
        seq_lens=seq.tolist(),
        seq_lens_tensor=seq_t,
        max_query_len=int(qlen.max()),
        max_prefill_seq_len=int(prefill_lens.max()) if prefill_lens.size else 0,
        max_decode_seq_len=int(decode_lens.max()) if decode_lens.size else 0,
        query_start_loc=qsl,
        seq_start_loc=ssl,
        context_lens_tensor=ctx_t,
        block_tables=bt_out,
        use_cuda_graph=False,
    )
    return toks, positions, metadata


def decode_requests(context_lens: Sequence[int], first_token: int = 0) -> List[Tuple]:
    """``RequestMeta`` tuples of a decode batch: request i holds
    ``context_lens[i]`` cached tokens and decodes one more."""
    return [(i, [first_token + i], int(c) + 1, int(c)) for i, c in enumerate(context_lens)]
