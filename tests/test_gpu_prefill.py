"""GPU parity of the varlen prefill attention (EXT flash_attn_varlen_func, the
prompt run reached from aegaeon/aegaeon/worker.py:517-523) against the
oracle's float64 textbook attention, through the C ABI.

Tolerance: the kernel rounds P to 16 bits before P.V, as FlashAttention does,
and rounds the output to the I/O dtype.  The output's own rounding already
costs ~1.6e-3 relative L2 in bf16 (~2.0e-4 in fp16) against float64, so a flat
2e-3 bar would leave P's rounding ~0.4e-3.  The bar is therefore the relative
L2 error of the float64 result rounded to the I/O dtype plus 1e-3 (bf16) /
1.5e-4 (fp16) for P's rounding (measured excess: at most 0.7e-3 / 0.09e-3),
and an elementwise error of at most 2^-7 (bf16) / 2^-9 (fp16) of the output's
largest magnitude (bf16: half the bar of the first version, twice the worst
error measured over these cases, 3.8e-3 of it)."""
import math

import numpy as np
import pytest
import torch

from aegaeon_amd import attention as A
from aegaeon_amd._lib import AegkvError
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu

BARS = {torch.bfloat16: (1e-3, 2.0 ** -7), torch.float16: (1.5e-4, 2.0 ** -9)}


def _packed(lens, Hq, Hkv, D, dtype, seed, extra=0):
    g = torch.Generator(device="cuda").manual_seed(seed)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    T = int(cu[-1]) + extra
    q = torch.randn((T, Hq, D), generator=g, device="cuda").to(dtype)
    k = torch.randn((T, Hkv, D), generator=g, device="cuda").to(dtype)
    v = torch.randn((T, Hkv, D), generator=g, device="cuda").to(dtype)
    return cu, q, k, v


def _check(got, q, k, v, cu, scale, causal, dtype, n_tokens=None):
    torch.cuda.synchronize()
    n = int(cu[-1]) if n_tokens is None else n_tokens
    ref = ko.varlen_prefill_attention(q[:n].double().cpu().numpy(), k[:n].double().cpu().numpy(),
                                      v[:n].double().cpu().numpy(), cu, scale, causal)
    return _within_bars(got[:n].double().cpu().numpy(), ref, dtype)


def _within_bars(out, ref, dtype):
    assert np.isfinite(out).all()
    extra, elem = BARS[dtype]
    nref = max(np.linalg.norm(ref), 1e-30)
    err = np.linalg.norm(out - ref) / nref
    rounding = np.linalg.norm(torch.from_numpy(ref).to(dtype).double().numpy() - ref) / nref
    worst = np.abs(out - ref).max() / max(np.abs(ref).max(), 1e-30)
    assert err <= rounding + extra, (err, rounding, worst)
    assert worst <= elem, (err, worst)
    return err


@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (8, 8, 64), (16, 2, 128), (12, 3, 64)])
@pytest.mark.parametrize("causal", [True, False])
def test_ragged_batch_matches_oracle(Hq, Hkv, D, causal):
    lens = [1, 15, 16, 17, 63, 64, 65, 127, 128, 129, 300]
    cu, q, k, v = _packed(lens, Hq, Hkv, D, torch.bfloat16, Hq + D)
    scale = 1.0 / math.sqrt(D)
    cu_t = torch.from_numpy(cu).cuda()
    out = A.varlen_prefill_attention(q, k, v, cu_t, max(lens), scale, causal)
    _check(out, q, k, v, cu, scale, causal, torch.bfloat16)


LONG_LENS = [1537, 1, 255, 256, 257, 2000, 64, 33]  # longest > 1536: the ping-pong kernel


@pytest.mark.parametrize("Hq,Hkv,D", [(8, 2, 128), (12, 3, 64)])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_prompts_match_oracle(Hq, Hkv, D, causal, dtype):
    """Batches whose longest prompt exceeds 1536 tokens run on the eight-wave
    ping-pong kernel (direct-to-LDS K/V, transposing V reads); lengths at and
    around the 64-key and 256-query tile edges, a 1-token prompt."""
    cu, q, k, v = _packed(LONG_LENS, Hq, Hkv, D, dtype, 31 + D)
    scale = 1.0 / math.sqrt(D)
    out = A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), max(LONG_LENS), scale,
                                     causal)
    _check(out, q, k, v, cu, scale, causal, dtype)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_and_short_kernels_bit_identical(D, causal, dtype):
    """The same prompts through both kernels: the exact host bound (1000,
    the four-wave kernel) and a loose bound of 2048 (the ping-pong kernel).
    Both accumulate every product in the same order, so the outputs are equal
    bit for bit; the short run is also checked against the oracle."""
    lens = [1000, 65, 1, 640, 129, 999]
    cu, q, k, v = _packed(lens, 8, 2, D, dtype, 77 + D)
    cu_t = torch.from_numpy(cu).cuda()
    short = A.varlen_prefill_attention(q, k, v, cu_t, max(lens), 0.09, causal)
    long = A.varlen_prefill_attention(q, k, v, cu_t, 2048, 0.09, causal)
    torch.cuda.synchronize()
    assert torch.equal(short.view(torch.int16), long.view(torch.int16))
    _check(short, q, k, v, cu, 0.09, causal, dtype)


def test_long_prompts_strided_views():
    """The ping-pong kernel on column slices of a fused QKV projection (token
    strides differ from the rows) with out a slice of a wider buffer."""
    Hq, Hkv, D = 28, 4, 128
    lens = [1800, 90]
    T = sum(lens)
    g = torch.Generator(device="cuda").manual_seed(13)
    qkv = torch.randn((T, (Hq + 2 * Hkv) * D), generator=g, device="cuda").to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(T, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
    wide = torch.full((T, Hq * D + 64), 7.0, device="cuda", dtype=torch.bfloat16)
    out = wide[:, :Hq * D].view(T, Hq, D)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), max(lens), 0.088, True,
                               out=out)
    _check(out, q, k, v, cu, 0.088, True, torch.bfloat16)
    assert bool((wide[:, Hq * D:] == 7.0).all())


@pytest.mark.parametrize("D", [64, 128])
def test_fp16(D):
    lens = [200, 7, 129]
    cu, q, k, v = _packed(lens, 8, 2, D, torch.float16, 5)
    cu_t = torch.from_numpy(cu).cuda()
    out = A.varlen_prefill_attention(q, k, v, cu_t, max(lens), 0.1, True)
    _check(out, q, k, v, cu, 0.1, True, torch.float16)


def test_strided_views_of_fused_qkv():
    """q, k, v as column slices of one [T, (Hq + 2 Hkv) D] projection output,
    out as a slice of a wider buffer: token strides differ from the rows."""
    Hq, Hkv, D = 28, 4, 128
    lens = [33, 190, 64]
    T = sum(lens)
    g = torch.Generator(device="cuda").manual_seed(11)
    qkv = torch.randn((T, (Hq + 2 * Hkv) * D), generator=g, device="cuda").to(torch.bfloat16)
    q = qkv[:, :Hq * D].view(T, Hq, D)
    k = qkv[:, Hq * D:(Hq + Hkv) * D].view(T, Hkv, D)
    v = qkv[:, (Hq + Hkv) * D:].view(T, Hkv, D)
    wide = torch.full((T, Hq * D + 64), 7.0, device="cuda", dtype=torch.bfloat16)
    out = wide[:, :Hq * D].view(T, Hq, D)
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int32)
    A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), max(lens), 0.088, True,
                               out=out)
    _check(out, q, k, v, cu, 0.088, True, torch.bfloat16)
    assert bool((wide[:, Hq * D:] == 7.0).all())


@pytest.mark.parametrize("bound", [400, 2048])  # the four-wave and the ping-pong kernel
def test_empty_sequences_loose_bound_and_nan_padding(bound):
    """Zero-length sequences, a host bound above every length, and NaN rows
    after the last sequence (padding tokens): the outputs of real tokens are
    right and padding rows of out are not written."""
    lens = [0, 40, 0, 130, 1]
    cu, q, k, v = _packed(lens, 4, 2, 64, torch.bfloat16, 3, extra=24)
    n = int(cu[-1])
    for x in (q, k, v):
        x[n:] = float("nan")
    out = torch.full_like(q, 3.0)
    A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), bound, 0.125, True, out=out)
    _check(out, q, k, v, cu, 0.125, True, torch.bfloat16)
    assert bool((out[n:] == 3.0).all())


def test_lengths_clamped_to_host_bound():
    """A device length above max_seqlen is clamped to it, never read past."""
    lens = [100, 50]
    cu, q, k, v = _packed(lens, 4, 4, 64, torch.bfloat16, 8)
    out = torch.zeros_like(q)
    A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), 64, 0.125, True, out=out)
    torch.cuda.synchronize()
    # sequence 0 is processed as its first 64 tokens; sequence 1 (50) in full
    ref0 = ko.varlen_prefill_attention(q[:64].double().cpu().numpy(),
                                       k[:64].double().cpu().numpy(),
                                       v[:64].double().cpu().numpy(), [0, 64], 0.125, True)
    got = out.double().cpu().numpy()
    assert np.abs(got[:64] - ref0).max() <= 2.0 ** -6 * np.abs(ref0).max()
    assert not got[64:100].any()
    _check(out[100:], q[100:], k[100:], v[100:], np.array([0, 50], dtype=np.int32), 0.125,
           True, torch.bfloat16)


@pytest.mark.parametrize("lens,heads", [
    ([300, 77], (28, 4, 128)), ([1200, 700, 1000, 333], (28, 4, 128)),  # four-wave
    ([2000, 300, 77, 700], (28, 4, 128)),                                # ping-pong
    ([2048] * 4, (16, 2, 64)),       # ping-pong at D = 64: two workgroups per CU
    ([256] * 32, (16, 2, 64))])      # four-wave at D = 64, several workgroups per CU
@pytest.mark.parametrize("causal", [True, False])
def test_deterministic(lens, heads, causal):
    """Repeated calls give the same bits (the register exchange between the
    wave halves included, also where two workgroups share a CU and their
    softmax waves a SIMD), and so does the other kernel on the same prompts
    (a host bound of 1536 or 2048).  The ragged four-wave batch deals its
    units round-robin over the XCDs, the co-residency under which scores read
    before their MFMAs finished once gave run-to-run differences."""
    Hq, Hkv, D = heads
    cu, q, k, v = _packed(lens, Hq, Hkv, D, torch.bfloat16, 12)
    cu_t = torch.from_numpy(cu).cuda()
    runs = [A.varlen_prefill_attention(q, k, v, cu_t, max(lens), 0.088, causal) for _ in range(5)]
    other = A.varlen_prefill_attention(q, k, v, cu_t, 1536 if max(lens) > 1536 else 2048, 0.088,
                                       causal)
    torch.cuda.synchronize()
    for r in runs[1:]:
        assert torch.equal(runs[0].view(torch.int16), r.view(torch.int16))
    if max(lens) <= 1536:  # a bound below the longest prompt clamps it: compare only then
        assert torch.equal(runs[0].view(torch.int16), other.view(torch.int16))


def test_qwen_prompt_batch_full_size():
    """Qwen2.5-7B prompt run, 4 prompts x 2048 tokens, GQA 28/4, D 128, bf16,
    against the float64 oracle at full size."""
    lens = [2048] * 4
    cu, q, k, v = _packed(lens, 28, 4, 128, torch.bfloat16, 21)
    scale = 1.0 / math.sqrt(128)
    out = A.flash_attn_varlen_func(q, k, v, torch.from_numpy(cu).cuda(),
                                   torch.from_numpy(cu).cuda(), 2048, 2048, softmax_scale=scale,
                                   causal=True)
    _check(out, q, k, v, cu, scale, True, torch.bfloat16)


def test_units_split_into_slices_over_xcds():
    """92 (prompt, head) units of up to 1536 tokens on the four-wave kernel:
    92 is not a multiple of the eight XCDs and each CU has several tiles, so
    every unit's tiles are dealt as two interleaved slices.  The output
    matches the oracle, and equals the ping-pong kernel's (a loose bound,
    whole units per XCD) bit for bit."""
    rng = np.random.default_rng(23)
    lens = rng.integers(1100, 1537, 23).tolist()
    lens[5] = 1536
    cu, q, k, v = _packed(lens, 4, 1, 64, torch.bfloat16, 23)
    cu_t = torch.from_numpy(cu).cuda()
    out = A.varlen_prefill_attention(q, k, v, cu_t, 1536, 0.125, True)
    other = A.varlen_prefill_attention(q, k, v, cu_t, 1537, 0.125, True)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), other.view(torch.int16))
    _check(out, q, k, v, cu, 0.125, True, torch.bfloat16)


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_32k_prompt_sampled_rows(causal, dtype):
    """A 32768-token prompt (128 query tiles of the ping-pong kernel) beside a
    300-token one, Qwen2.5-7B heads.  The full float64 textbook is out of
    reach at this length, so sampled query rows are checked, each against the
    oracle's decode attention of that query over the keys it sees (keys 0..r
    of its prompt when causal, all of them otherwise), with the prompt's K/V
    laid out as 16-token blocks: tile edges, the middle and the last rows."""
    lens = [32768, 300]
    Hq, Hkv, D = 28, 4, 128
    cu, q, k, v = _packed(lens, Hq, Hkv, D, dtype, 41)
    scale = 1.0 / math.sqrt(D)
    out = A.varlen_prefill_attention(q, k, v, torch.from_numpy(cu).cuda(), max(lens), scale,
                                     causal)
    torch.cuda.synchronize()
    rng = np.random.default_rng(41)
    rows = [(0, r) for r in [0, 1, 63, 64, 255, 256, 257, 1535, 1536, 4095, 16383, 16384,
                             32766, 32767]]
    rows += [(0, int(r)) for r in rng.integers(0, lens[0], 6)] + [(1, 0), (1, 17), (1, 299)]
    T = int(cu[-1])
    nblk = -(-T // 16)
    kf = np.zeros((nblk * 16, Hkv, D))
    vf = np.zeros((nblk * 16, Hkv, D))
    kf[:T] = k.double().cpu().numpy()
    vf[:T] = v.double().cpu().numpy()
    tables, seen, idx = [], [], []
    for b, r in rows:
        first = int(cu[b]) // 16  # every prompt starts on a 16-token boundary here
        tables.append(list(range(first, first + -(-lens[b] // 16))))
        seen.append(r + 1 if causal else lens[b])
        idx.append(int(cu[b]) + r)
    ref = ko.paged_decode_attention(q[idx].double().cpu().numpy(),
                                    kf.reshape(nblk, 16, Hkv, D), vf.reshape(nblk, 16, Hkv, D),
                                    ko.pad_block_tables(tables), seen, scale)
    _within_bars(out[idx].double().cpu().numpy(), ref, dtype)


def test_wrapper_rejects_unsupported_options():
    cu, q, k, v = _packed([10], 4, 4, 64, torch.bfloat16, 1)
    cu_t = torch.from_numpy(cu).cuda()
    with pytest.raises(NotImplementedError):
        A.flash_attn_varlen_func(q, k, v, cu_t, cu_t, 10, 10, dropout_p=0.1)
    with pytest.raises(NotImplementedError):
        A.flash_attn_varlen_func(q, k, v, cu_t, cu_t, 10, 10, window_size=(4, 0))
    with pytest.raises(NotImplementedError):
        A.flash_attn_varlen_func(q, k, v, cu_t, cu_t, 10, 12)
    with pytest.raises(AegkvError):
        A.varlen_prefill_attention(q[:, :, :32].contiguous(), k[:, :, :32].contiguous(),
                                   v[:, :, :32].contiguous(), cu_t, 10, 0.1)
