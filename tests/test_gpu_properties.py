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
