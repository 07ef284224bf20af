"""Property tests over random batches on the GPU, through the C ABI, against
the oracle (hypothesis, derandomized so every run draws the same cases).

* Decode attention (flash_attn_with_kvcache semantics, selected at
  aegaeon/aegaeon/worker.py:410-418): random batches of 1-10 sequences,
  lengths biased to block and tile edges, every supported head shape and
  dtype, random workgroup counts.  The unplanned call is within the float64
  oracle's tolerance, the planned call equals it bit for bit, and the
  appending call equals reshape_and_cache_flash followed by the attention,
  output and cache.
* Varlen prefill attention (flash_attn_varlen_func, reached from
  worker.py:517-523): random ragged prompt batches, causal or not, bf16 and
  fp16.  The output is within the float64 oracle's bars, and the two kernels
  (a host bound above 1536 tokens selects the ping-pong kernel) agree bit for
  bit.
* Byte movers: one decode token per sequence appended into every layer of a
  random pool (EXT reshape_and_cache_flash, per layer through the storage
  view), padding and out-of-pool slots skipped, then a random layer range
  de-paged; a random live set compacted by the defrag kernel; all bit-exact.
* Step inputs (worker.py:596-676): random prefill/decode mixes, equal to the
  oracle's restatement of the host loops.

The tolerances are the ones the per-op test files state; their checks are
reused here.
"""
import math

import numpy as np
import pytest
import torch
from hypothesis import HealthCheck, given, settings, strategies as st

from aegaeon_amd import attention as A
from oracle import kv_oracle as ko
from tests.kvtest_utils import to_bits
from tests.test_gpu_attention import _check as decode_check
from tests.test_gpu_prefill import _check as prefill_check

pytestmark = pytest.mark.gpu

_SETTINGS = dict(deadline=None, derandomize=True, database=None,
                 suppress_health_check=[HealthCheck.too_slow,
                                        HealthCheck.function_scoped_fixture])
_TORCH = {"bf16": torch.bfloat16, "fp16": torch.float16}

DECODE_HEADS = [(28, 4, 128), (32, 4, 128), (8, 8, 128), (16, 1, 64), (6, 2, 256), (12, 6, 128),
                (8, 2, 64), (40, 40, 128)]


@st.composite
def _decode_case(draw):
    n = draw(st.integers(1, 10))
    edge = st.sampled_from([0, 1, 2, 15, 16, 17, 31, 32, 33, 255, 256, 257, 1023, 1024, 1025])
    lens = draw(st.lists(st.one_of(st.integers(0, 2500), edge), min_size=n, max_size=n))
    if max(lens) == 0:
        lens[0] = 1
    heads = draw(st.sampled_from(DECODE_HEADS))
    dtype = draw(st.sampled_from(["bf16", "fp16"]))
    nwg = draw(st.one_of(st.just(0), st.integers(1, 600)))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return lens, heads, dtype, nwg, seed


@settings(max_examples=60, **_SETTINGS)
@given(case=_decode_case())
def test_decode_attention_random_batches(device, case):
    lens, (Hq, Hkv, D), dtype, nwg, seed = case
    lens = np.asarray(lens, dtype=np.int64)
    rng = np.random.default_rng(seed)
    need = [-(-int(x) // 16) for x in lens]
    N = sum(need) + 4
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    gen = torch.Generator(device=device).manual_seed(seed)
    tdt = _TORCH[dtype]
    storage = torch.randn((N, 1, 2, 16, Hkv, D), generator=gen, device=device).to(tdt)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    kc, vc = view[0, 0], view[0, 1]
    q = torch.randn((len(lens), Hq, D), generator=gen, device=device).to(tdt)
    bt = torch.from_numpy(padded).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    ml = int(lens.max())
    scale = 1.0 / math.sqrt(D)

    out = A.paged_decode_attention(q, kc, vc, bt, sl, scale, ml, n_workgroups=nwg)
    plan = A.DecodePlan(bt, sl, ml, Hkv, nwg)
    planned = A.paged_decode_attention(q, kc, vc, None, None, scale, ml, n_workgroups=nwg,
                                       plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(planned.view(torch.int16), out.view(torch.int16))
    oracle = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), dtype),
                                       ko.bits_to_float(to_bits(kc), dtype),
                                       ko.bits_to_float(to_bits(vc), dtype), padded, lens, scale)
    decode_check(to_bits(out), oracle, dtype)

    # the non-empty sequences with their last token appended by the call itself
    live = np.nonzero(lens)[0]
    key = torch.randn((len(live), Hkv, D), generator=gen, device=device).to(tdt)
    val = torch.randn((len(live), Hkv, D), generator=gen, device=device).to(tdt)
    slots = ko.slot_mapping([tables[i] for i in live], lens[live] - 1, lens[live])
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[0, 0], view2[0, 1],
                              torch.from_numpy(slots).to(device))
    li = torch.from_numpy(live).to(device)
    ql, btl, sll = q[li].contiguous(), bt[li].contiguous(), sl[li].contiguous()
    ref = A.paged_decode_attention(ql, view2[0, 0], view2[0, 1], btl, sll, scale, ml,
                                   n_workgroups=nwg)
    got = A.paged_decode_attention(ql, kc, vc, btl, sll, scale, ml, n_workgroups=nwg, key=key,
                                   value=val)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))


PREFILL_HEADS = [(8, 2, 128), (4, 4, 64), (6, 3, 64), (6, 1, 128)]


@st.composite
def _prefill_case(draw):
    n = draw(st.integers(1, 4))
    edge = st.sampled_from([0, 1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 255, 256, 257, 1535,
                            1536, 1537])
    lens = draw(st.lists(st.one_of(st.integers(0, 1700), edge), min_size=n, max_size=n))
    if max(lens) == 0:
        lens[0] = 1
    heads = draw(st.sampled_from(PREFILL_HEADS))
    causal = draw(st.booleans())
    dtype = draw(st.sampled_from(["bf16", "fp16"]))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return lens, heads, causal, dtype, seed


@settings(max_examples=40, **_SETTINGS)
@given(case=_prefill_case())
def test_prefill_random_batches(device, case):
    lens, (Hq, Hkv, D), causal, dtype, seed = case
    tdt = _TORCH[dtype]
    gen = torch.Generator(device=device).manual_seed(seed)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1])
    q = torch.randn((T, Hq, D), generator=gen, device=device).to(tdt)
    k = torch.randn((T, Hkv, D), generator=gen, device=device).to(tdt)
    v = torch.randn((T, Hkv, D), generator=gen, device=device).to(tdt)
    cu_t = torch.from_numpy(cu).to(device)
    scale = 1.0 / math.sqrt(D)
    out = A.varlen_prefill_attention(q, k, v, cu_t, max(lens), scale, causal)
    other = A.varlen_prefill_attention(q, k, v, cu_t, max(1537, max(lens)), scale, causal)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), other.view(torch.int16))
    prefill_check(out, q, k, v, cu, scale, causal, tdt)


# ------------------------------------------------------------------ byte movers
@st.composite
def _append_case(draw):
    L = draw(st.integers(1, 4))
    Hkv = draw(st.sampled_from([1, 2, 4, 8]))
    D = draw(st.sampled_from([64, 128, 256]))
    n = draw(st.integers(1, 12))
    edge = st.sampled_from([1, 15, 16, 17, 32, 33])
    lens = draw(st.lists(st.one_of(st.integers(1, 300), edge), min_size=n, max_size=n))
    # per token: 0 its own slot, 1 vLLM's padding slot -1, 2 a slot past the pool
    kinds = draw(st.lists(st.sampled_from([0, 0, 0, 1, 2]), min_size=n, max_size=n))
    extra = draw(st.integers(0, 40))
    first = draw(st.integers(0, L - 1))
    count = draw(st.integers(1, L - first))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return L, Hkv, D, lens, kinds, extra, (first, count), seed


def _random_bits_on(device, shape, seed):
    g = torch.Generator(device=device).manual_seed(seed)
    return torch.randint(-2 ** 15, 2 ** 15, shape, dtype=torch.int16, generator=g,
                         device=device)


@settings(max_examples=40, **_SETTINGS)
@given(case=_append_case())
def test_append_then_gather_random_pools(device, case):
    """One decode token per sequence appended into every layer of a random
    [N, L, 2, 16, Hkv, D] pool in one launch (padding slots -1 and slots past
    the pool skipped), then a random layer range de-paged: both bit-exact
    against the oracle, NaN bit patterns included."""
    L, Hkv, D, lens, kinds, extra, (first, count), seed = case
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    need = [-(-int(x) // 16) for x in lens]
    N = sum(need) + extra + 1
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    slots = ko.slot_mapping(tables, lens - 1, lens)
    kinds = np.asarray(kinds)
    slots[kinds == 1] = -1
    slots[kinds == 2] = N * 16 + rng.integers(0, 1000, int((kinds == 2).sum()))
    storage = _random_bits_on(device, (N, L, 2, 16, Hkv, D), seed)
    key = _random_bits_on(device, (L, len(lens), Hkv, D), seed + 1)
    val = _random_bits_on(device, (L, len(lens), Hkv, D), seed + 2)
    ref = storage.cpu().numpy().view(np.uint16).copy()
    # the oracle writes every slot >= 0; a slot past the pool is skipped like -1
    ko.append_layers(key.cpu().numpy().view(np.uint16), val.cpu().numpy().view(np.uint16), ref,
                     np.where(slots >= N * 16, -1, slots))
    bf = torch.bfloat16
    cache = storage.view(bf)
    A.append_kv(key.view(bf), val.view(bf), cache, torch.from_numpy(slots).to(device))
    torch.cuda.synchronize()
    assert np.array_equal(storage.cpu().numpy().view(np.uint16), ref)

    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    out_k, out_v = A.gather_tokens(cache, bt, sl, int(lens.sum()), int(lens.max()),
                                   layers=(first, count))
    rk, rv = ko.gather_tokens(ref, tables, lens, layers=list(range(first, first + count)))
    assert np.array_equal(to_bits(out_k), rk)
    assert np.array_equal(to_bits(out_v), rv)


@st.composite
def _defrag_case(draw):
    bb = draw(st.sampled_from([16, 4096, 16400, 65536, 131072]))
    n = draw(st.integers(2, 300))
    live = draw(st.lists(st.integers(0, n - 1), min_size=0, max_size=n, unique=True))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return bb, n, live, seed


@settings(max_examples=30, **_SETTINGS)
@given(case=_defrag_case())
def test_defrag_random_pools(device, case):
    """A random live set of a pool of n blocks compacted into its dense
    prefix: the move lists equal the oracle's, the moved blocks land bit for
    bit, every other block keeps its bytes, and the rewritten tables equal the
    oracle's."""
    from aegaeon_amd.pool import plan_compaction, remap_tables
    bb, n, live, seed = case
    src, dst = plan_compaction(live, list(range(n)))
    osrc, odst = ko.plan_defrag(live, list(range(n)))
    assert list(src) == osrc and list(dst) == odst
    pool = _random_bits_on(device, (n * bb // 2,), seed)
    ref = pool.cpu().numpy().view(np.uint8).reshape(n, bb).copy()
    ref[np.asarray(odst, dtype=np.int64)] = ref[np.asarray(osrc, dtype=np.int64)]
    from aegaeon_amd import ops
    ops.defrag_blocks(pool.view(torch.uint8), src, dst, block_bytes=bb)
    torch.cuda.synchronize()
    assert np.array_equal(pool.cpu().numpy().view(np.uint8).reshape(n, bb), ref)
    rng = np.random.default_rng(seed)
    order = rng.permutation(len(live)).tolist()
    tables = [[live[i] for i in order[j::3]] for j in range(3)]
    assert remap_tables(tables, src, dst) == ko.apply_defrag(tables, osrc, odst)


@st.composite
def _inputs_case(draw):
    n_prefill = draw(st.integers(0, 6))
    n_decode = draw(st.integers(0 if n_prefill else 1, 40))
    edge = st.sampled_from([1, 15, 16, 17, 31, 32, 33])
    prompt = st.one_of(st.integers(1, 400), edge)
    ctxs = st.one_of(st.integers(1, 3000), edge)
    prefills = draw(st.lists(prompt, min_size=n_prefill, max_size=n_prefill))
    decodes = draw(st.lists(ctxs, min_size=n_decode, max_size=n_decode))
    spare = draw(st.lists(st.integers(0, 2), min_size=n_prefill + n_decode,
                          max_size=n_prefill + n_decode))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return prefills, decodes, spare, seed


@settings(max_examples=40, **_SETTINGS)
@given(case=_inputs_case())
def test_prepare_inputs_random_batches(device, case):
    """Random prefill/decode mixes with tables drawn from a permutation of
    the pool (some holding spare pre-allocated blocks): every output of the
    device-side preparation equals the oracle's restatement of the worker's
    host loops, values and dtypes."""
    from aegaeon_amd import inputs as I
    from tests.test_gpu_inputs import _compare
    prefills, decodes, spare, seed = case
    rng = np.random.default_rng(seed)
    perm = iter(rng.permutation(1 << 16).tolist())
    reqs, tables = [], []
    for i, n in enumerate(prefills):
        reqs.append((i, rng.integers(0, 32000, n).tolist(), n, 0))
        tables.append([next(perm) for _ in range(-(-n // 16) + spare[i])])
    for j, ctx in enumerate(decodes):
        i = len(prefills) + j
        reqs.append((i, [int(rng.integers(0, 32000))], ctx + 1, ctx))
        tables.append([next(perm) for _ in range(-(-(ctx + 1) // 16) + spare[i])])
    _compare(I.prepare_model_inputs(reqs, tables, device), ko.prepare_model_inputs(reqs, tables))
