"""The C ABI without a GPU: libaegkv.so loads, exports every function that
include/aegkv.h declares, and rejects bad arguments on the host with the
documented status codes before any HIP call is made (pointers here are host
addresses that the library never dereferences on these paths)."""
import ctypes
import re

import numpy as np
import pytest

from aegaeon_amd import _lib

OK, INVALID, RANGE, MISALIGNED, OVERLAP, DUP, UNSUP, WS = 0, -1, -2, -3, -4, -5, -6, -7


@pytest.fixture(scope="module")
def lib():
    return _lib.load()


def _i64(a):
    a = np.ascontiguousarray(np.asarray(a, dtype=np.int64))
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def _buf(nbytes, misalign=0):
    raw = np.zeros(nbytes + 64, dtype=np.uint8)
    base = raw.ctypes.data
    addr = (base + 15) // 16 * 16 + misalign
    return raw, addr


def test_every_declared_symbol_is_exported_and_typed(lib):
    declared = _lib.declared_symbols()
    assert len(declared) >= 12
    assert set(declared) == set(_lib.SIGNATURES), "ctypes table and header disagree"
    for name in declared:
        assert hasattr(lib, name), name


def test_header_status_codes_match_strerror(lib):
    text = _lib.HEADER_PATH.read_text()
    codes = {m[0]: int(m[1]) for m in re.findall(r"#define (AEGKV_(?:OK|ERR_\w+)) \(?(-?\d+)\)?", text)}
    assert codes["AEGKV_OK"] == OK and codes["AEGKV_ERR_WORKSPACE"] == WS
    msgs = {c: _lib.strerror(c) for c in codes.values()}
    assert len(set(msgs.values())) == len(msgs)  # every code has its own message
    assert "unknown" in _lib.strerror(-99)
    assert lib.aegkv_version() >> 16 == 1


def test_block_copy_argument_checks(lib):
    raw, pool = _buf(16 * 64)
    s, sp = _i64([0, 1, 2])
    d, dp = _i64([3, 4, 5])
    bad, badp = _i64([0, 64, 1])
    dup, dupp = _i64([6, 6, 7])
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, dp, -1, 16, None) == INVALID
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, dp, 0, 16, None) == OK  # no-op
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, badp, dp, 3, 16, None) == RANGE
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, badp, 3, 16, None) == RANGE
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, dupp, 3, 16, None) == DUP
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, sp, 3, 16, None) == OVERLAP
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, dp, 3, 24, None) == MISALIGNED
    raw2, mis = _buf(16 * 64, misalign=8)
    assert lib.aegkv_copy_blocks(mis, 64, pool, 64, sp, dp, 3, 16, None) == MISALIGNED
    # partially aliased distinct pools would make the order matter
    assert lib.aegkv_copy_blocks(pool, 64, pool + 16, 63, sp, dp, 3, 16, None) == OVERLAP
    assert lib.aegkv_defrag_blocks(pool, 64, sp, sp, 3, 16, None) == OVERLAP
    assert lib.aegkv_defrag_blocks(pool, 64, None, dp, 3, 16, None) == INVALID
    assert lib.aegkv_pack_blocks(pool, 64, None, 3, pool, 16, None) == INVALID
    assert lib.aegkv_scatter_blocks(pool, badp, 3, pool, 64, 16, None) == RANGE
    # the last id of the pool, repeated (the checks mark a bitmap over the pool)
    top, topp = _i64([63, 62, 63])
    assert lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, topp, 3, 16, None) == DUP
    # a pool far larger than the lists: the checks sort copies instead
    huge = 1 << 40
    assert lib.aegkv_copy_blocks(pool, huge, pool, huge, sp, dupp, 3, 16, None) == DUP
    assert lib.aegkv_copy_blocks(pool, huge, pool, huge, sp, sp, 3, 16, None) == OVERLAP
    assert lib.aegkv_defrag_blocks(pool, huge, sp, sp, 3, 16, None) == OVERLAP
    # a pool whose byte size does not fit 64 bits
    assert lib.aegkv_copy_blocks(pool, 1 << 62, pool + 4096, 64, sp, dp, 3, 16, None) == INVALID
    # the checks leave no marks behind: after the rejected calls above, lists
    # that reuse their ids pass them (and the call then fails later, at the
    # device query, as there is no GPU here)
    ok, okp = _i64([6, 7, 63])
    rc = lib.aegkv_copy_blocks(pool, 64, pool, 64, sp, okp, 3, 16, None)
    assert rc not in (OK, DUP, OVERLAP, RANGE, INVALID, MISALIGNED), rc


def test_swap_argument_checks(lib):
    raw, dev = _buf(16 * 8)
    host = np.zeros(16 * 8, dtype=np.uint8)
    s, sp = _i64([0, 1])
    big, bigp = _i64([0, 8])
    dup, dupp = _i64([2, 2])
    h = host.ctypes.data
    assert lib.aegkv_swap_blocks(sp, sp, -1, 0, dev, 8, h, 8, 16, None, 0, None) == INVALID
    assert lib.aegkv_swap_blocks(sp, sp, 0, 0, dev, 8, h, 8, 16, None, 0, None) == OK
    assert lib.aegkv_swap_blocks(None, sp, 2, 0, dev, 8, h, 8, 16, None, 0, None) == INVALID
    assert lib.aegkv_swap_blocks(bigp, sp, 2, 0, dev, 8, h, 8, 16, None, 0, None) == RANGE
    assert lib.aegkv_swap_blocks(sp, bigp, 2, 1, dev, 8, h, 8, 16, None, 0, None) == RANGE
    assert lib.aegkv_swap_blocks(sp, dupp, 2, 0, dev, 8, h, 8, 16, None, 0, None) == DUP
    assert lib.aegkv_swap_blocks(sp, sp, 2, 0, dev, 8, h, 8, 0, None, 0, None) == INVALID
    # a host pool whose byte size does not fit 64 bits
    assert lib.aegkv_swap_blocks(sp, sp, 2, 0, dev, 8, h, 1 << 62, 16, None, 0, None) == INVALID


def test_bounced_swap_argument_checks(lib):
    raw, dev = _buf(16 * 8)
    host = np.zeros(16 * 8, dtype=np.uint8)
    h = host.ctypes.data
    rawb, bnc = _buf(16 * 4)
    raws, stg = _buf(16 * 4)
    s, sp = _i64([0, 1])
    big, bigp = _i64([0, 8])
    dup, dupp = _i64([2, 2])
    sw = lib.aegkv_swap_blocks_bounced

    def call(src=sp, dst=sp, n=2, swap_in=0, dev_=dev, n_dev=8, n_host=8, bb=16, staging=stg,
             stg_bytes=64, bounce=bnc, bounce_bytes=64):
        return sw(src, dst, n, swap_in, dev_, n_dev, h, n_host, bb, staging, stg_bytes, bounce,
                  bounce_bytes, None)

    assert call(n=-1) == INVALID
    assert call(n=0) == OK
    assert call(bounce=None) == INVALID
    assert call(staging=None) == INVALID
    assert call(src=None) == INVALID
    assert call(src=bigp) == RANGE
    assert call(dst=bigp, swap_in=1) == RANGE
    assert call(dst=dupp) == DUP
    assert call(bb=24) == MISALIGNED
    assert call(bounce_bytes=8) == WS       # the bounce buffer holds no block
    assert call(stg_bytes=8) == WS          # nor does the staging buffer
    assert call(n_host=1 << 62) == INVALID  # a pool whose byte size does not fit 64 bits


def test_append_and_gather_argument_checks(lib):
    raw, p = _buf(4096)
    raw2, mis = _buf(4096, misalign=2)
    args = dict(n_tokens=4, n_layers=1, bs=16, H=2, D=64, eb=2)

    def append(key=p, elem=2, tok_stride=128, n_layers=1, n_tokens=4, heads=2, dim=64):
        return lib.aegkv_kv_append(key, p, tok_stride, 128, 0, 0, p, n_tokens, p, p, 4096, 0, 4,
                                   n_layers, 16, heads, dim, elem, None)

    assert append(elem=4) == UNSUP
    assert append(n_layers=0) == INVALID
    assert append(n_tokens=0) == OK
    assert append(key=mis) == MISALIGNED
    assert append(tok_stride=3) == MISALIGNED
    assert append(dim=3) == MISALIGNED  # 2*3*2 = 12-byte rows
    assert append(n_tokens=1 << 62) == UNSUP  # 2^67 chunks: no product may wrap
    # gather: max_seq_len needs more blocks than the table is wide
    assert lib.aegkv_gather_tokens(p, p, 4096, 0, 4, p, 1, p, p, 2, 40, p, p, 80, 0, 1, 16, 2,
                                   64, 2, None) == INVALID
    assert lib.aegkv_gather_tokens(p, p, 4096, 0, 4, p, 3, p, p, 2, 40, p, p, 80, 0, 1, 16, 2,
                                   64, 4, None) == UNSUP
    assert lib.aegkv_gather_tokens(p, p, 4096, 0, 4, p, 3, p, p, 0, 40, p, p, 80, 0, 1, 16, 2,
                                   64, 2, None) == OK
    # rows wider than 2 GiB
    assert lib.aegkv_gather_tokens(p, p, 4096, 0, 4, p, 3, p, p, 2, 40, p, p, 80, 0, 1, 16,
                                   1 << 16, 1 << 16, 2, None) == UNSUP
    del args


def test_attention_argument_checks_and_workspace_size(lib):
    raw, p = _buf(1 << 16)
    ws = lib.aegkv_paged_decode_attention_workspace_size
    # (batch, Hq, Hkv, D, max_seq_len, dtype, n_workgroups); an explicit
    # workgroup count sizes the workspace without a device query
    assert ws(0, 28, 4, 128, 4096, 0, 8) == 0
    assert ws(4, 28, 4, 100, 4096, 0, 8) == UNSUP
    assert ws(4, 30, 4, 128, 4096, 0, 8) == INVALID
    assert ws(4, 28, 4, 128, 4096, 9, 8) == UNSUP
    assert ws(4, 28, 4, 128, 4096, 0, -1) == INVALID
    # one 16-byte descriptor per workgroup, then (n_wg + groups*batch) slots
    # of hpg = 4 * 7 query heads: float2 (m, l) and D floats each
    up = lambda x: -(-x // 256) * 256  # noqa: E731
    cnt = up(8 * 16)
    slots = 8 + 1 * 4
    want = cnt + up(slots * 28 * 8) + up(slots * 28 * 128 * 4)
    assert ws(4, 28, 4, 128, 4096, 0, 8) == want
    assert ws(4, 28, 4, 128, 4096, 0, 16) > want
    # Llama-shaped 40/40: ten groups of four kv heads, one query head each
    slots = 8 + 10 * 4
    assert ws(4, 40, 40, 128, 4096, 1, 8) == cnt + up(slots * 4 * 8) + up(slots * 4 * 128 * 4)
    assert ws(4, 28, 4, 128, 4096, 0, 8193) == UNSUP
    # batches above 2048 are launched in chunks of 2048 sharing one workspace
    assert ws(5000, 28, 4, 128, 4096, 0, 8) == ws(2048, 28, 4, 128, 4096, 0, 8)

    def attn(Hq=28, Hkv=4, D=128, bs=16, dtype=0, max_len=64, max_blocks=4, wsp=None, wsb=0,
             nwg=0, q=p):
        return lib.aegkv_paged_decode_attention(p, Hq * D, q, Hq * D, p, p, 16 * Hkv * D, 8, p,
                                                max_blocks, p, 2, max_len, Hq, Hkv, D, bs, 0.1,
                                                dtype, nwg, wsp, wsb, None)

    assert attn(Hq=30) == INVALID
    assert attn(D=96) == UNSUP
    assert attn(bs=32) == UNSUP
    assert attn(dtype=7) == UNSUP
    assert attn(Hq=34, Hkv=2) == UNSUP  # group of 17 > 16
    assert attn(max_len=100) == INVALID  # needs 7 blocks, table has 4
    assert attn(nwg=-1) == INVALID
    assert attn(nwg=8193) == UNSUP
    need = ws(2, 28, 4, 128, 4096, 0, 1)
    assert need > 0
    assert attn(max_len=4096, max_blocks=256, nwg=1) == WS
    assert attn(max_len=4096, max_blocks=256, nwg=1, wsp=p, wsb=need - 1) == WS
    raw2, mis = _buf(64, misalign=4)
    assert attn(q=mis) == MISALIGNED


def test_decode_plan_host_checks(lib):
    """Plan sizing and the host checks of plan building and planned calls
    (explicit workgroup counts: no device query, no launch)."""
    raw, p = _buf(1 << 20)
    size = lib.aegkv_paged_decode_plan_size
    up = lambda x: -(-x // 256) * 256  # noqa: E731
    # (batch, Hkv, max_seq_len, n_workgroups): records of 8 int32, descriptors,
    # 64 first ids and 64 first tags per workgroup, one last-block id per
    # sequence, then batch * ceil(max_seq_len / 16) ids and as many tags
    assert size(0, 4, 4096, 8) == 0
    assert size(3, 4, 100, 8) == (up(8 * 32) + up(8 * 16) + up(8 * 512) + up(3 * 4)
                                  + 2 * up(3 * 7 * 4))
    assert size(2049, 4, 100, 8) == UNSUP  # one launch's batch at most
    assert size(3, 0, 100, 8) == INVALID
    assert size(3, 4, -1, 8) == INVALID
    assert size(3, 4, 100, 8193) == UNSUP
    plan = lib.aegkv_paged_decode_plan
    # (tables, max_blocks, seq_lens, batch, max_seq_len, Hkv, nwg, plan, plan_bytes, stream)
    need = size(3, 4, 100, 8)
    assert plan(p, 7, p, 3, 100, 4, 8, p, need - 1, None) == INVALID
    assert plan(p, 6, p, 3, 100, 4, 8, p, need, None) == INVALID  # tables narrower than 100 tokens
    assert plan(None, 7, p, 3, 100, 4, 8, p, need, None) == INVALID
    raw2, mis = _buf(need + 64, misalign=4)
    assert plan(p, 7, p, 3, 100, 4, 8, mis, need, None) == MISALIGNED
    assert plan(p, 7, p, 0, 100, 4, 8, None, 0, None) == 0  # empty batch: nothing to do

    def planned(batch=2, plan_ptr=p, plan_bytes=1 << 16, max_len=64):
        return lib.aegkv_paged_decode_attention_planned(
            p, 28 * 128, p, 28 * 128, p, p, 16 * 4 * 128, 8, plan_ptr, plan_bytes, p, batch,
            max_len, 28, 4, 128, 16, 0.1, 0, 8, p, 1 << 20, None)

    assert planned(plan_ptr=None) == INVALID
    assert planned(plan_bytes=size(2, 4, 64, 8) - 1) == INVALID
    assert planned(batch=2049, max_len=16) == UNSUP


def test_prepare_inputs_host_checks(lib):
    """Argument errors are found on the host, before any device work."""
    raw, p = _buf(1 << 12)
    i32 = lambda xs: np.asarray(xs, dtype=np.int32)  # noqa: E731
    i64 = lambda xs: np.asarray(xs, dtype=np.int64)  # noqa: E731

    def prep(ids, offs, seq, ctx, n_query, batch=None, pad=4, bs=16):
        ids, offs, seq, ctx = i32(ids), i64(offs), i32(seq), i32(ctx)
        toks = i64(np.zeros(max(n_query, 1)))
        b = len(seq) if batch is None else batch
        return lib.aegkv_prepare_inputs(ids.ctypes.data if ids.size else None, offs.ctypes.data,
                                        seq.ctypes.data, ctx.ctypes.data, toks.ctypes.data, b,
                                        bs, pad, p, p, p, p, p, p, p, p, n_query, None)

    assert prep([1], [0, 1], [5], [6], 0) == INVALID          # context_len > seq_len
    assert prep([1], [0, 1], [17], [16], 1) == RANGE   # position 16 needs a 2nd block
    assert prep([1, 2], [0, 2], [17], [16], 2) == INVALID     # query tokens must total 1
    assert prep([1, 2], [0, 2], [17], [16], 1, pad=1) == INVALID  # decode table wider than pad
    assert prep([-1], [0, 1], [3], [0], 3) == RANGE    # negative block id
    assert prep([1], [1, 1], [3], [0], 3) == INVALID          # offsets must start at 0
    assert prep([], [0], [], [], 0, batch=0) == OK
    assert prep([1], [0, 1], [3], [0], 3, bs=0) == INVALID


def test_prefill_attention_host_checks(lib):
    """Shapes, dtypes, strides and alignment are checked on the host."""
    raw, p = _buf(1 << 12)

    def call(q=p, out=p, qs=28 * 128, ks=4 * 128, os_=28 * 128, batch=1, ms=16, total=16,
             hq=28, hkv=4, d=128, dt=0, scale=0.1):
        return lib.aegkv_varlen_prefill_attention(out, os_, q, qs, p, ks, p, ks, p, batch, ms,
                                                  total, hq, hkv, d, scale, 1, dt, None)

    assert call(hq=28, hkv=5) == INVALID           # Hq not a multiple of Hkv
    assert call(d=32) == UNSUP                      # head_dim 64 or 128 only
    assert call(dt=7) == UNSUP
    assert call(qs=27 * 128) == INVALID             # token row shorter than its heads
    assert call(os_=28 * 128 + 4) == MISALIGNED     # stride not a multiple of 16 bytes
    assert call(q=p + 2) == MISALIGNED
    assert call(scale=float("nan")) == INVALID
    assert call(batch=0, q=None, out=None) == OK    # nothing to do
    assert call(ms=0) == OK
    assert call(q=None) == INVALID


def test_fused_append_host_checks(lib):
    """The appending attention rejects a missing or misaligned new row and a
    batch stride shorter than one token's rows, before any launch."""
    raw, p = _buf(1 << 20)
    f = lib.aegkv_paged_decode_attention_append
    Hq, Hkv, D = 8, 4, 128

    def call(key=p, kstride=Hkv * D, value=p, vstride=Hkv * D):
        # out, q, key, value, caches, tables, lengths: host addresses never read here
        return f(p, Hq * D, p, Hq * D, key, kstride, value, vstride, p, p, 16 * Hkv * D, 8, p, 4,
                 p, 2, 64, Hq, Hkv, D, 16, 0.1, 0, 8, p, 1 << 20, None)

    assert call(key=None) == INVALID
    assert call(value=None) == INVALID
    assert call(kstride=Hkv * D - 8) == INVALID
    assert call(key=p + 8) == MISALIGNED
    assert call(vstride=Hkv * D + 4) == MISALIGNED
    g = lib.aegkv_paged_decode_attention_append_planned
    assert g(p, Hq * D, p, Hq * D, None, Hkv * D, p, Hkv * D, p, p, 16 * Hkv * D, 8, p, 1 << 20,
             p, 2, 64, Hq, Hkv, D, 16, 0.1, 0, 8, p, 1 << 20, None) == INVALID


def test_signal_arrays_reject_bad_arguments_on_the_host(lib):
    words, n = ctypes.c_void_p(), ctypes.c_int64()
    handle = (ctypes.c_char * 64)()
    assert lib.aegkv_signals_create(0, ctypes.byref(words), handle) == INVALID
    assert lib.aegkv_signals_create((1 << 20) + 1, ctypes.byref(words), handle) == INVALID
    assert lib.aegkv_signals_create(4, None, handle) == INVALID
    assert lib.aegkv_signals_open(None, ctypes.byref(words), ctypes.byref(n)) == INVALID
    assert lib.aegkv_signals_open(handle, ctypes.byref(words), None) == INVALID
    assert lib.aegkv_signals_destroy(None) == INVALID
    assert lib.aegkv_signals_close(None) == INVALID
    raw, addr = _buf(64, misalign=4)
    assert lib.aegkv_signal_set(addr, 1, None) == INVALID       # not 8-byte aligned
    assert lib.aegkv_signal_wait(addr, 1, 10, None, None) == INVALID
    raw2, addr2 = _buf(64)
    assert lib.aegkv_signal_wait(addr2, 1, 0, None, None) == INVALID  # zero timeout
