"""GPU parity of paged GQA decode attention (vllm-flash-attn flash_attn_with_kvcache
semantics, selected at aegaeon/aegaeon/worker.py:410-418).

Tolerance (written here, from the path's requirement): the bf16/fp16 output
must be within 2e-3 relative L2 error of the float64 textbook result computed
from the same 16-bit inputs, overall; and every element within one ulp of the
output dtype at the reference value plus 1e-5 absolute (fp32 accumulation
leaves only the final rounding, which can land on either neighbour near a tie;
the absolute term covers fp32 summation error on outputs near zero).  The
kernel's P.V product carries each softmax weight to 16 significant bits (a
high and a low 16-bit part), so a weight's relative error is at most 2^-17
and an output's absolute error beyond its final rounding at most
2^-17 * max|v|; batches large enough to meet that bound on an element near
zero pass that absolute term instead of 1e-5.
"""
import math

import numpy as np
import pytest
import torch

from aegaeon_amd import attention as A
from aegaeon_amd.workloads import qwen_attention_batch
from oracle import kv_oracle as ko
from tests.kvtest_utils import bf16_ulp, fp16_ulp, random_bits, to_bits, to_device_bits

pytestmark = pytest.mark.gpu

REL_L2 = 2e-3


def _setup(rng, lens, Hq, Hkv, D, dtype, N=None, pad_to=None):
    lens = np.asarray(lens, dtype=np.int64)
    need = [-(-int(x) // 16) for x in lens]
    N = N or max(8, 2 * sum(need) + 3)
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    if pad_to is not None and padded.shape[1] < pad_to:
        padded = np.pad(padded, ((0, 0), (0, pad_to - padded.shape[1])))
    kc = random_bits(rng, (N, 16, Hkv, D), dtype)
    vc = random_bits(rng, (N, 16, Hkv, D), dtype)
    q = random_bits(rng, (len(lens), Hq, D), dtype)
    return lens, tables, padded, q, kc, vc


def _check(out_bits, ref, dtype, abs_tol=1e-5):
    got = ko.bits_to_float(out_bits, dtype)
    err = np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30)
    assert err <= REL_L2, f"relative L2 error {err:.3e}"
    ulp = bf16_ulp(ref) if dtype == "bf16" else fp16_ulp(ref)
    bad = np.abs(got - ref) > ulp + abs_tol
    assert not bad.any(), f"{int(bad.sum())} elements beyond 1 ulp; max {np.abs(got-ref)[bad].max()}"
    return err


def _run(device, lens, Hq, Hkv, D, dtype, nwg=0, seed=0, kc_override=None):
    rng = np.random.default_rng(seed)
    lens, tables, padded, q, kc, vc = _setup(rng, lens, Hq, Hkv, D, dtype)
    if kc_override is not None:
        kc, vc = kc_override(kc, vc, tables, lens)
    scale = 1.0 / math.sqrt(D)
    out = A.paged_decode_attention(
        to_device_bits(q, dtype, device), to_device_bits(kc, dtype, device),
        to_device_bits(vc, dtype, device), torch.from_numpy(padded).to(device),
        torch.from_numpy(lens.astype(np.int32)).to(device), scale, int(lens.max()),
        n_workgroups=nwg)
    ref = ko.paged_decode_attention(ko.bits_to_float(q, dtype), ko.bits_to_float(kc, dtype),
                                    ko.bits_to_float(vc, dtype), padded, lens, scale)
    return to_bits(out), ref, (lens, tables, padded, q, kc, vc)


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (32, 4, 128), (8, 8, 128), (16, 1, 64),
                                      (6, 2, 256), (12, 6, 128), (40, 40, 128)])
@pytest.mark.parametrize("nwg", [0, 1, 3, 64, 1000])
def test_matches_fp64_textbook(device, dtype, Hq, Hkv, D, nwg):
    """Every workgroup count partitions the same blocks differently (one
    workgroup walking all sequences; pieces of a few blocks; more workgroups
    than blocks); the result must not depend on it."""
    lens = [1, 15, 16, 17, 31, 64, 200, 517, 0, 1100]
    out, ref, _ = _run(device, lens, Hq, Hkv, D, dtype, nwg=nwg, seed=Hq * 1000 + D + nwg)
    _check(out, ref, dtype)


def test_batch_above_one_launch(device):
    """2500 sequences run as launches of 2048 and 452 sharing one workspace."""
    rng = np.random.default_rng(11)
    lens = rng.integers(0, 70, size=2500)
    out, ref, _ = _run(device, lens, 8, 2, 64, "bf16", seed=11)
    _check(out, ref, "bf16")


def test_len_one_returns_v0_exactly(device):
    out, ref, (lens, tables, padded, q, kc, vc) = _run(device, [1, 1, 1], 28, 4, 128, "bf16")
    for b, t in enumerate(tables):
        v0 = vc[t[0], 0]  # [Hkv, D]
        assert np.array_equal(out[b].reshape(4, 7, 128), np.repeat(v0[:, None, :], 7, axis=1))


def test_identical_keys_give_mean_of_values(device):
    def same_keys(kc, vc, tables, lens):
        kc = kc.copy()
        kc[:] = kc[0, 0][None, None]  # every token has the same key
        return kc, vc
    out, ref, (lens, tables, padded, q, kc, vc) = _run(device, [40, 77], 28, 4, 128, "bf16",
                                                      kc_override=same_keys)
    for b, ln in enumerate(lens):
        nb = -(-int(ln) // 16)
        v = ko.bits_to_float(vc[tables[b][:nb]], "bf16").reshape(nb * 16, 4, 128)[:ln]
        mean = v.mean(axis=0)  # [Hkv, D]
        got = ko.bits_to_float(out[b], "bf16").reshape(4, 7, 128)
        assert np.allclose(got, mean[:, None, :], rtol=8e-3, atol=8e-3)


def test_dominant_logit_selects_its_value(device):
    """One key aligned with a large multiple of q dominates: out ~= V_argmax."""
    rng = np.random.default_rng(1)
    Hq = Hkv = 2
    D = 128
    lens = np.asarray([50], dtype=np.int64)
    lens, tables, padded, q, kc, vc = _setup(rng, lens, Hq, Hkv, D, "bf16")
    qf = ko.bits_to_float(q, "bf16")
    kf = ko.bits_to_float(kc, "bf16") * 0.01
    hot = 37
    blk, off = tables[0][hot // 16], hot % 16
    kf[blk, off] = qf[0] * 4.0  # per kv head h: key = 4 q_h -> logit 4|q|^2/sqrt(D) >> others
    kc = ko.float_to_bits(kf, "bf16")
    out = A.paged_decode_attention(
        to_device_bits(q, "bf16", device), to_device_bits(kc, "bf16", device),
        to_device_bits(vc, "bf16", device), torch.from_numpy(padded).to(device),
        torch.from_numpy(lens.astype(np.int32)).to(device), 1 / math.sqrt(D), 50)
    got = ko.bits_to_float(to_bits(out), "bf16")[0]
    want = ko.bits_to_float(vc[blk, off], "bf16")
    assert np.allclose(got, want, rtol=1e-2, atol=1e-2)


def test_stale_rows_and_padding_blocks_never_read(device):
    """NaN in the unused rows of each tail block and in the 0-padded table
    entries' block (id 0) must not reach the output (worker.py:640-646)."""
    rng = np.random.default_rng(4)
    lens = np.asarray([5, 33, 16], dtype=np.int64)
    lens, tables, padded, q, kc, vc = _setup(rng, lens, 28, 4, 128, "bf16", N=40)
    used = {x for t in tables for x in t}
    free0 = 0 if 0 not in used else None
    nan = ko.float_to_bits(np.float32(np.nan), "bf16")
    for b, ln in enumerate(lens):
        last = tables[b][-1]
        kc[last, int(ln) % 16 or 16:] = nan
        vc[last, int(ln) % 16 or 16:] = nan
    if free0 is not None:
        kc[0] = nan
        vc[0] = nan
    padded = np.pad(padded, ((0, 0), (0, 4)))  # extra 0 ids past every sequence
    scale = 1 / math.sqrt(128)
    out = A.paged_decode_attention(
        to_device_bits(q, "bf16", device), to_device_bits(kc, "bf16", device),
        to_device_bits(vc, "bf16", device), torch.from_numpy(padded).to(device),
        torch.from_numpy(lens.astype(np.int32)).to(device), scale, int(padded.shape[1] * 16))
    got = to_bits(out)
    assert not np.isnan(ko.bits_to_float(got, "bf16")).any()
    ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(kc, "bf16"),
                                    ko.bits_to_float(vc, "bf16"), padded, lens, scale)
    _check(got, ref, "bf16")


def test_zero_length_gives_zeros(device):
    out, ref, _ = _run(device, [0, 20], 28, 4, 128, "bf16")
    assert not ko.bits_to_float(out[0], "bf16").any()
    _check(out[1:], ref[1:], "bf16")


def test_flash_attn_with_kvcache_surface(device):
    rng = np.random.default_rng(2)
    lens, tables, padded, q, kc, vc = _setup(rng, [70, 3], 28, 4, 128, "bf16")
    qt = to_device_bits(q, "bf16", device).view(2, 1, 28, 128)
    out = A.flash_attn_with_kvcache(qt, to_device_bits(kc, "bf16", device),
                                    to_device_bits(vc, "bf16", device),
                                    block_table=torch.from_numpy(padded).to(device),
                                    cache_seqlens=torch.from_numpy(lens.astype(np.int32)).to(device))
    assert out.shape == (2, 1, 28, 128)
    ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(kc, "bf16"),
                                    ko.bits_to_float(vc, "bf16"), padded, lens, 1 / math.sqrt(128))
    _check(to_bits(out).reshape(2, 28, 128), ref, "bf16")


def test_qwen_full_batch_layer(device):
    """The Qwen2.5-7B decode batch (128 sequences, lognormal mean 1500, up to
    8192 tokens) for one layer of a pool sized 2x the need; every sequence is
    checked against the float64 oracle."""
    wb = qwen_attention_batch(0)
    g = wb.geometry
    rng = np.random.default_rng(0)
    N = wb.n_pool_blocks
    used = sorted({x for t in wb.block_tables for x in t})
    remap = {x: i for i, x in enumerate(used)}
    k_used = random_bits(rng, (len(used), 16, g.n_kv_heads, g.head_dim), "bf16")
    v_used = random_bits(rng, (len(used), 16, g.n_kv_heads, g.head_dim), "bf16")
    kc = np.zeros((N, *k_used.shape[1:]), dtype=np.uint16)
    vc = np.zeros_like(kc)
    kc[used] = k_used
    vc[used] = v_used
    q = random_bits(rng, (wb.batch, g.n_q_heads, g.head_dim), "bf16")
    lens = wb.seq_lens
    padded = wb.padded_tables()
    compact = ko.pad_block_tables([[remap[x] for x in t] for t in wb.block_tables])
    scale = 1 / math.sqrt(g.head_dim)
    out = A.paged_decode_attention(
        to_device_bits(q, "bf16", device), to_device_bits(kc, "bf16", device),
        to_device_bits(vc, "bf16", device), torch.from_numpy(padded).to(device),
        torch.from_numpy(lens.astype(np.int32)).to(device), scale, int(lens.max()))
    ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(k_used, "bf16"),
                                    ko.bits_to_float(v_used, "bf16"), compact, lens, scale)
    _check(to_bits(out), ref, "bf16")


def test_workspace_reused_across_calls(device):
    """One workspace serves consecutive calls of different batches: nothing a
    call leaves in it may leak into the next (stale partials, descriptors)."""
    ws = A.attention_workspace(8, 28, 4, 128, 2000, torch.bfloat16, n_workgroups=5,
                               device=device)
    ws.fill_(0x7F)  # stale bytes: the result must not depend on the contents
    for seed, lens in ((21, [900, 3, 1500, 40, 0, 17, 700, 2000]),
                       (22, [1, 2, 3, 4]),
                       (21, [900, 3, 1500, 40, 0, 17, 700, 2000])):
        rng = np.random.default_rng(seed)
        lens, tables, padded, q, kc, vc = _setup(rng, lens, 28, 4, 128, "bf16", pad_to=125)
        scale = 1.0 / math.sqrt(128)
        out = A.paged_decode_attention(
            to_device_bits(q, "bf16", device), to_device_bits(kc, "bf16", device),
            to_device_bits(vc, "bf16", device), torch.from_numpy(padded).to(device),
            torch.from_numpy(lens.astype(np.int32)).to(device), scale, 2000, n_workgroups=5,
            workspace=ws)
        ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(kc, "bf16"),
                                        ko.bits_to_float(vc, "bf16"), padded, lens, scale)
        _check(to_bits(out), ref, "bf16")


def _device_case(device, lens, Hq, Hkv, D, dtype, seed, pad_to=None):
    rng = np.random.default_rng(seed)
    lens, tables, padded, q, kc, vc = _setup(rng, lens, Hq, Hkv, D, dtype, pad_to=pad_to)
    return (lens, padded, q, kc, vc, to_device_bits(q, dtype, device),
            to_device_bits(kc, dtype, device), to_device_bits(vc, dtype, device),
            torch.from_numpy(padded).to(device),
            torch.from_numpy(lens.astype(np.int32)).to(device))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (16, 1, 64), (6, 2, 256), (12, 6, 128),
                                      (40, 40, 128)])
@pytest.mark.parametrize("nwg", [0, 1, 3, 64, 1000])
def test_planned_call_is_bit_identical(device, dtype, Hq, Hkv, D, nwg):
    """A decode plan reproduces the split the kernel computes for itself (the
    same pieces, merged the same way): the planned call's output equals the
    unplanned one bit for bit, for every workgroup count (one workgroup over
    all sequences and all kv-head groups; more workgroups than blocks)."""
    lens = [1, 15, 16, 17, 31, 64, 200, 517, 0, 1100]
    _, _, _, _, _, q, kc, vc, bt, sl = _device_case(device, lens, Hq, Hkv, D, dtype, nwg + D)
    scale = 1.0 / math.sqrt(D)
    ref = A.paged_decode_attention(q, kc, vc, bt, sl, scale, 1100, n_workgroups=nwg)
    plan = A.DecodePlan(bt, sl, 1100, Hkv, nwg)
    got = A.paged_decode_attention(q, kc, vc, None, None, scale, 1100, n_workgroups=nwg,
                                   plan=plan)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_plan_serves_every_layer(device):
    """One plan per step, many layers: each layer's queries and caches differ,
    the tables and lengths do not.  Every planned output equals the unplanned
    call and the float64 oracle."""
    rng = np.random.default_rng(31)
    lens = rng.integers(1, 3000, size=40)
    lens[[3, 17]] = 0
    lens, tables, padded, _, _, _ = _setup(rng, lens, 28, 4, 128, "bf16")
    bt = torch.from_numpy(padded).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    ml = int(lens.max())
    plan = A.DecodePlan(bt, sl, ml, 4)
    scale = 1.0 / math.sqrt(128)
    N = max(8, 2 * int(sum(-(-int(x) // 16) for x in lens)) + 3)
    for layer in range(3):
        q = random_bits(rng, (40, 28, 128), "bf16")
        kc = random_bits(rng, (N, 16, 4, 128), "bf16")
        vc = random_bits(rng, (N, 16, 4, 128), "bf16")
        qd, kd, vd = (to_device_bits(x, "bf16", device) for x in (q, kc, vc))
        got = A.paged_decode_attention(qd, kd, vd, bt, sl, scale, ml, plan=plan)
        ref = A.paged_decode_attention(qd, kd, vd, bt, sl, scale, ml)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), layer
        oracle = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(kc, "bf16"),
                                           ko.bits_to_float(vc, "bf16"), padded, lens, scale)
        _check(to_bits(got), oracle, "bf16")


def test_plan_qwen_full_batch(device):
    """The Qwen2.5-7B decode batch through a plan, against the unplanned call."""
    wb = qwen_attention_batch(0)
    g = wb.geometry
    gen = torch.Generator(device=device).manual_seed(5)
    kc = torch.randn((wb.n_pool_blocks, 16, 4, 128), generator=gen, device=device).to(torch.bfloat16)
    vc = torch.randn(kc.shape, generator=gen, device=device).to(torch.bfloat16)
    q = torch.randn((wb.batch, 28, 128), generator=gen, device=device).to(torch.bfloat16)
    bt = torch.from_numpy(wb.padded_tables()).to(device)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(device)
    ml = int(wb.seq_lens.max())
    plan = A.DecodePlan(bt, sl, ml, g.n_kv_heads)
    got = A.paged_decode_attention(q, kc, vc, bt, sl, 1 / math.sqrt(128), ml, plan=plan)
    ref = A.paged_decode_attention(q, kc, vc, bt, sl, 1 / math.sqrt(128), ml)
    torch.cuda.synchronize()
    assert torch.equal(got, ref)


def test_plan_misuse_is_rejected(device):
    lens = [40, 7]
    _, _, _, _, _, q, kc, vc, bt, sl = _device_case(device, lens, 8, 2, 64, "bf16", 3)
    plan = A.DecodePlan(bt, sl, 40, 2)
    with pytest.raises(ValueError):  # another max_seq_len
        A.paged_decode_attention(q, kc, vc, None, None, 0.125, 64, plan=plan)
    with pytest.raises(ValueError):  # another workgroup count
        A.paged_decode_attention(q, kc, vc, None, None, 0.125, 40, n_workgroups=3, plan=plan)
    with pytest.raises(ValueError):  # tables the plan was not built from
        A.paged_decode_attention(q, kc, vc, bt.clone(), sl, 0.125, 40, plan=plan)
    big = torch.zeros((2500, 1), dtype=torch.int32, device=device)
    with pytest.raises(A._lib.AegkvError):  # above one launch's batch
        A.DecodePlan(big, torch.ones(2500, dtype=torch.int32, device=device), 16, 2)


def test_yi_decode_after_unified_pool_defrag(device):
    """The unified-pool decode step at full size: a 44 GiB byte pool of bf16
    values co-hosting three models, the Yi-1.5-9B blocks compacted into their
    dense prefix, then layer 0's decode attention for the 64 Yi sequences
    (GQA 32/4, lognormal mean 1000) through a plan over the rewritten tables,
    read from the reference's [N, L, 2, 16, Hkv, D] storage as a strided view.
    Checked against the float64 oracle on the K/V taken before the moves,
    through the original tables."""
    from aegaeon_amd import ops
    from aegaeon_amd.pool import plan_compaction, remap_tables
    from aegaeon_amd.workloads import unified_pool_workload
    wl = unified_pool_workload(0)
    g = wl.geometries[wl.decode_model]
    bb = g.block_bytes
    torch.cuda.empty_cache()
    if torch.cuda.get_device_properties(device).total_memory < wl.pool_bytes + (16 << 30):
        pytest.skip("needs %d GiB of device memory" % ((wl.pool_bytes >> 30) + 16))
    gen = torch.Generator(device=device).manual_seed(7)
    pool = torch.empty(wl.pool_bytes, dtype=torch.uint8, device=device)
    pool.view(torch.bfloat16).normal_(generator=gen)
    nb = wl.pool_bytes // bb
    typed = pool[:nb * bb].view(torch.bfloat16).view(nb, *g.block_shape)
    old_tables = wl.tables[wl.decode_model]
    used = sorted({b for t in old_tables for b in t})
    idx = torch.tensor(used, device=device)
    k_used = to_bits(typed[idx, 0, 0])                  # layer 0, K: [n, 16, Hkv, D]
    v_used = to_bits(typed[idx, 0, 1])
    src, dst = plan_compaction([b for t in old_tables for b in t],
                               wl.valid_ids(wl.decode_model))
    ops.defrag_blocks(pool, src, dst, block_bytes=bb)
    tables = remap_tables(old_tables, src, dst)
    lens = np.asarray(wl.yi_context_lens, dtype=np.int64)
    q = torch.randn((len(lens), g.n_q_heads, g.head_dim), generator=gen,
                    device=device).to(torch.bfloat16)
    view = typed.permute(1, 2, 0, 3, 4, 5)
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    ml = int(lens.max())
    scale = 1 / math.sqrt(g.head_dim)
    plan = A.DecodePlan(bt, sl, ml, g.n_kv_heads)
    out = A.paged_decode_attention(q, view[0, 0], view[0, 1], None, None, scale, ml, plan=plan)
    torch.cuda.synchronize()
    pos = {b: i for i, b in enumerate(used)}
    compact = ko.pad_block_tables([[pos[b] for b in t] for t in old_tables])
    ref = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), "bf16"),
                                    ko.bits_to_float(k_used, "bf16"),
                                    ko.bits_to_float(v_used, "bf16"), compact, lens, scale)
    _check(to_bits(out), ref, "bf16")
    del pool, typed, view
    torch.cuda.empty_cache()


def test_bad_inputs_raise_before_launch(device):
    """Host-side checks: every tensor the kernels read or write must be on the
    call's GPU, with the dtype the ABI reads it as; a host pointer never
    reaches a kernel."""
    lens = [40, 7]
    _, _, _, _, _, q, kc, vc, bt, sl = _device_case(device, lens, 8, 2, 64, "bf16", 4)
    ws = A.attention_workspace(2, 8, 2, 64, 40, torch.bfloat16)   # default device: the GPU
    assert ws is not None and ws.is_cuda and ws.device == device
    ok = A.paged_decode_attention(q, kc, vc, bt, sl, 0.125, 40, workspace=ws)
    torch.cuda.synchronize()
    cases = {
        "cpu workspace": dict(workspace=torch.empty(ws.numel(), dtype=torch.uint8)),
        "cpu block_tables": dict(block_tables=bt.cpu()),
        "cpu seq_lens": dict(seq_lens=sl.cpu()),
        "out of another dtype": dict(out=torch.empty(q.shape, dtype=torch.float16,
                                                     device=device)),
        "cpu out": dict(out=torch.empty(q.shape, dtype=q.dtype)),
        "tables of another batch": dict(block_tables=bt[:1]),
    }
    for name, kw in cases.items():
        args = dict(block_tables=bt, seq_lens=sl, workspace=ws)
        args.update(kw)
        with pytest.raises(ValueError):
            A.paged_decode_attention(q, kc, vc, args.pop("block_tables"), args.pop("seq_lens"),
                                     0.125, 40, **args)
        torch.cuda.synchronize()
    with pytest.raises(ValueError):
        A.attention_workspace(2, 8, 2, 64, 40, torch.bfloat16, device="cpu")
    again = A.paged_decode_attention(q, kc, vc, bt, sl, 0.125, 40, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(again, ok)


def test_plan_built_on_another_stream(device):
    """A plan built on one stream and used on another: the call's stream waits
    for the build (the plan kernel is held back behind a spin on its stream,
    so without the wait the attention would read an unwritten plan)."""
    lens = [300, 1, 4000, 77, 0, 1500, 16, 2049]
    lens, padded, q_b, kc_b, vc_b, q, kc, vc, bt, sl = _device_case(device, lens, 28, 4, 128,
                                                                  "bf16", 41)
    ref = A.paged_decode_attention(q, kc, vc, bt, sl, 1 / math.sqrt(128), 4000)
    torch.cuda.synchronize()
    build, use = torch.cuda.Stream(device=device), torch.cuda.Stream(device=device)
    for trial in range(3):
        with torch.cuda.stream(build):
            torch.cuda._sleep(20_000_000)           # tens of ms on the build stream
            plan = A.DecodePlan(bt, sl, 4000, 4)
        with torch.cuda.stream(use):
            got = A.paged_decode_attention(q, kc, vc, None, None, 1 / math.sqrt(128), 4000,
                                           plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(got, ref), trial


def test_yi_decode_step_after_unified_pool_defrag(device):
    """The whole decode step of the unified-pool workload at full size: after
    the Yi-1.5-9B compaction, one token per sequence is appended to every one
    of the 48 layers of the compacted pool (slots through the rewritten
    tables, worker.py:628-633), then attention over ctx + 1 tokens runs for
    layers 0 and 47 through a plan over the rewritten tables.  The pool after
    the append equals the pool before it with the oracle's append applied to
    the touched blocks (bit for bit, so nothing else changed), and attention
    matches the float64 oracle on the K/V taken before the moves plus the
    appended token."""
    from aegaeon_amd import ops
    from aegaeon_amd.pool import plan_compaction, remap_tables
    from aegaeon_amd.workloads import unified_pool_workload
    wl = unified_pool_workload(0)
    g = wl.geometries[wl.decode_model]
    bb = g.block_bytes
    torch.cuda.empty_cache()
    if torch.cuda.get_device_properties(device).total_memory < 2 * wl.pool_bytes + (16 << 30):
        pytest.skip("needs %d GiB of device memory" % ((2 * wl.pool_bytes >> 30) + 16))
    gen = torch.Generator(device=device).manual_seed(9)
    pool = torch.empty(wl.pool_bytes, dtype=torch.uint8, device=device)
    pool.view(torch.bfloat16).normal_(generator=gen)
    nb = wl.pool_bytes // bb
    typed = pool[:nb * bb].view(torch.bfloat16).view(nb, *g.block_shape)
    old_tables = wl.tables[wl.decode_model]
    used = sorted({b for t in old_tables for b in t})
    pos = {b: i for i, b in enumerate(used)}
    idx = torch.tensor(used, device=device)
    layers = (0, g.n_layers - 1)
    kv_before = {l: (to_bits(typed[idx, l, 0]), to_bits(typed[idx, l, 1])) for l in layers}
    src, dst = plan_compaction([b for t in old_tables for b in t],
                               wl.valid_ids(wl.decode_model))
    ops.defrag_blocks(pool, src, dst, block_bytes=bb)
    tables = remap_tables(old_tables, src, dst)
    ctx = np.asarray(wl.yi_context_lens, dtype=np.int64)
    B = len(ctx)
    # the append: one token per sequence and layer at position ctx
    key = torch.randn((g.n_layers, B, g.n_kv_heads, g.head_dim), generator=gen,
                      device=device).to(torch.bfloat16)
    val = torch.randn(key.shape, generator=gen, device=device).to(torch.bfloat16)
    slots = ko.slot_mapping(tables, ctx, [c + 1 for c in ctx])
    targets = sorted({int(s) // 16 for s in slots})
    tidx = torch.tensor(targets, device=device)
    snapshot = pool.clone()
    expect = to_bits(typed[tidx])                       # [n_target, L, 2, 16, Hkv, D]
    tpos = {b: i for i, b in enumerate(targets)}
    compact_slots = np.asarray([tpos[int(s) // 16] * 16 + int(s) % 16 for s in slots],
                               dtype=np.int64)
    ko.append_layers(to_bits(key), to_bits(val), expect, compact_slots)
    A.append_kv(key, val, typed, torch.from_numpy(slots).to(device))
    torch.cuda.synchronize()
    snap_typed = snapshot[:nb * bb].view(torch.bfloat16).view(nb, *g.block_shape)
    snap_typed[tidx] = to_device_bits(expect, "bf16", device)
    assert torch.equal(pool, snapshot)                  # the append and nothing else
    del snapshot, snap_typed
    # attention over ctx + 1 through the rewritten tables, one plan for the step
    lens = ctx + 1
    view = typed.permute(1, 2, 0, 3, 4, 5)
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    ml = int(lens.max())
    scale = 1 / math.sqrt(g.head_dim)
    plan = A.DecodePlan(bt, sl, ml, g.n_kv_heads)
    compact = ko.pad_block_tables([[pos[b] for b in t] for t in old_tables])
    kb, vb = to_bits(key), to_bits(val)
    for l in layers:
        q = torch.randn((B, g.n_q_heads, g.head_dim), generator=gen,
                        device=device).to(torch.bfloat16)
        out = A.paged_decode_attention(q, view[l, 0], view[l, 1], None, None, scale, ml,
                                       plan=plan)
        torch.cuda.synchronize()
        k_ref, v_ref = (x.copy() for x in kv_before[l])
        for b in range(B):                               # the appended token, pre-move ids
            blk = pos[old_tables[b][int(ctx[b]) // 16]]
            k_ref[blk, int(ctx[b]) % 16] = kb[l, b]
            v_ref[blk, int(ctx[b]) % 16] = vb[l, b]
        ref = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), "bf16"),
                                        ko.bits_to_float(k_ref, "bf16"),
                                        ko.bits_to_float(v_ref, "bf16"), compact, lens, scale)
        _check(to_bits(out), ref, "bf16")
    del pool, typed, view
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# append fused into the attention (flash_attn_with_kvcache with k=, v=)
# ---------------------------------------------------------------------------
def _fused_case(device, lens, L, Hq, Hkv, D, dtype, seed):
    """A 6-d storage [N, L, 2, 16, Hkv, D] with scattered tables for
    sequences of `lens` tokens (the last one is the new token), the new rows
    and the slots the reference's slot mapping gives them."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int64)
    need = [-(-int(x) // 16) for x in lens]
    N = 2 * sum(need) + 5
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    storage = to_device_bits(random_bits(rng, (N, L, 2, 16, Hkv, D), dtype), dtype, device)
    key = to_device_bits(random_bits(rng, (len(lens), Hkv, D), dtype), dtype, device)
    val = to_device_bits(random_bits(rng, (len(lens), Hkv, D), dtype), dtype, device)
    q = to_device_bits(random_bits(rng, (len(lens), Hq, D), dtype), dtype, device)
    slots = ko.slot_mapping(tables, lens - 1, lens)
    return (lens, tables, storage, key, val, q,
            torch.from_numpy(ko.pad_block_tables(tables)).to(device),
            torch.from_numpy(lens.astype(np.int32)).to(device),
            torch.from_numpy(slots).to(device))


@pytest.mark.parametrize("dtype", ["bf16", "fp16"])
@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (16, 1, 64), (6, 2, 256), (40, 40, 128)])
@pytest.mark.parametrize("nwg", [0, 1, 7, 300])
@pytest.mark.parametrize("planned", [False, True])
def test_fused_append_equals_append_then_attention(device, dtype, Hq, Hkv, D, nwg, planned):
    """The fused call's output and cache equal reshape_and_cache_flash
    followed by the attention, bit for bit (new tokens at block offsets 0, 15
    and in between, a one-token sequence, sequences split across
    workgroups), and the output is within the float64 oracle's tolerance."""
    lens = [1, 16, 17, 32, 33, 200, 517, 1100, 15, 64 * 16 + 1]
    L, layer = 3, 1
    lens, tables, storage, key, val, q, bt, sl, slots = _fused_case(device, lens, L, Hq, Hkv, D,
                                                                    dtype, nwg + D + Hq)
    ml = int(lens.max())
    scale = 1.0 / math.sqrt(D)
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[layer, 0], view2[layer, 1], slots)
    plan = A.DecodePlan(bt, sl, ml, Hkv, nwg) if planned else None
    ref = A.paged_decode_attention(q, view2[layer, 0], view2[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    got = A.paged_decode_attention(q, view[layer, 0], view[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan, key=key, value=val)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))
    kb = to_bits(two[:, layer, 0])
    vb = to_bits(two[:, layer, 1])
    oracle = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), dtype),
                                       ko.bits_to_float(kb, dtype), ko.bits_to_float(vb, dtype),
                                       ko.pad_block_tables(tables), lens, scale)
    _check(to_bits(got), oracle, dtype)


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("nwg", [0, 5])
def test_fused_append_with_bound_below_longest(device, planned, nwg):
    """A host bound below the longest lengths: the fused call writes each new
    row at its own slot and attends the first max_seq_len cached tokens of the
    longer sequences, exactly as reshape_and_cache_flash followed by the
    bounded attention (no cached token is overwritten by a clamped row)."""
    lens = [1, 16, 17, 200, 299, 300, 301, 517, 1100]
    L, layer, Hq, Hkv, D = 2, 1, 28, 4, 128
    lens, tables, storage, key, val, q, bt, sl, slots = _fused_case(device, lens, L, Hq, Hkv, D,
                                                                    "bf16", 61 + nwg)
    ml = 300
    scale = 1.0 / math.sqrt(D)
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[layer, 0], view2[layer, 1], slots)
    plan = A.DecodePlan(bt, sl, ml, Hkv, nwg) if planned else None
    ref = A.paged_decode_attention(q, view2[layer, 0], view2[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    got = A.paged_decode_attention(q, view[layer, 0], view[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan, key=key, value=val)
    torch.cuda.synchronize()
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    kb = to_bits(two[:, layer, 0])
    vb = to_bits(two[:, layer, 1])
    oracle = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), "bf16"),
                                       ko.bits_to_float(kb, "bf16"), ko.bits_to_float(vb, "bf16"),
                                       ko.pad_block_tables(tables), np.minimum(lens, ml), scale)
    _check(to_bits(got), oracle, "bf16")


@pytest.mark.parametrize("planned", [False, True])
@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (16, 2, 64)])
@pytest.mark.parametrize("nwg", [1, 3, 0])
def test_fused_append_many_sequence_ends_per_range(device, planned, Hq, Hkv, D, nwg):
    """Ranges that end far more sequences than the kernel keeps new rows for
    at once (600 short sequences over 1 and 3 workgroups, ~100 per workgroup
    on the default grid), runs of empty sequences longer than the 64
    sequences one staging looks ahead over, and sequences longer than the
    host bound: output and cache equal reshape_and_cache_flash followed by the
    attention, bit for bit, and the output is within the float64 oracle's
    tolerance."""
    rng = np.random.default_rng(71 + nwg + D)
    B = 600
    lens = rng.integers(1, 40, B).astype(np.int64)
    lens[rng.random(B) < 0.2] = 0
    lens[100:180] = 0          # 80 empty sequences in a row
    lens[300:370] = 0
    lens[5], lens[450] = 700, 900
    ml = 512                   # sequences 5 and 450 exceed it
    need = [-(-int(x) // 16) for x in lens]
    N = 2 * sum(need) + 5
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    L, layer, dtype = 2, 1, "bf16"
    storage = to_device_bits(random_bits(rng, (N, L, 2, 16, Hkv, D), dtype), dtype, device)
    key = to_device_bits(random_bits(rng, (B, Hkv, D), dtype), dtype, device)
    val = to_device_bits(random_bits(rng, (B, Hkv, D), dtype), dtype, device)
    q = to_device_bits(random_bits(rng, (B, Hq, D), dtype), dtype, device)
    # the new token of sequence b at position len - 1; an empty one has none
    slots = np.array([t[(n - 1) // 16] * 16 + (n - 1) % 16 if n > 0 else -1
                      for t, n in zip(tables, lens)], dtype=np.int64)
    padded = ko.pad_block_tables([t if t else [0] for t in tables])
    bt = torch.from_numpy(padded).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    scale = 1.0 / math.sqrt(D)
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[layer, 0], view2[layer, 1],
                              torch.from_numpy(slots).to(device))
    plan = A.DecodePlan(bt, sl, ml, Hkv, nwg) if planned else None
    ref = A.paged_decode_attention(q, view2[layer, 0], view2[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    got = A.paged_decode_attention(q, view[layer, 0], view[layer, 1], bt, sl, scale, ml,
                                   n_workgroups=nwg, plan=plan, key=key, value=val)
    torch.cuda.synchronize()
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    kb = to_bits(two[:, layer, 0])
    vb = to_bits(two[:, layer, 1])
    oracle = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), dtype),
                                       ko.bits_to_float(kb, dtype), ko.bits_to_float(vb, dtype),
                                       padded, np.minimum(lens, ml), scale)
    # 2.15M outputs over up to 512 tokens: the P-precision bound of the header
    _check(to_bits(got), oracle, dtype,
           abs_tol=2.0 ** -17 * float(np.abs(ko.bits_to_float(vb, dtype)).max()))


def test_flash_attn_with_kvcache_table_without_room(device):
    """cache_seqlens at the table's capacity: the new token has no block, so
    nothing is written and the attention covers the cached tokens, as the
    default bound (the table's capacity) says; sequences with room append."""
    ctx = np.asarray([32, 5, 31], dtype=np.int64)        # tables of 2 blocks each
    rng = np.random.default_rng(62)
    N = 9
    ids = rng.permutation(N)[:6]
    tables = [[int(ids[0]), int(ids[1])], [int(ids[2]), int(ids[3])], [int(ids[4]), int(ids[5])]]
    storage = to_device_bits(random_bits(rng, (N, 1, 2, 16, 2, 64), "bf16"), "bf16", device)
    key = to_device_bits(random_bits(rng, (3, 1, 2, 64), "bf16"), "bf16", device)
    val = to_device_bits(random_bits(rng, (3, 1, 2, 64), "bf16"), "bf16", device)
    q = to_device_bits(random_bits(rng, (3, 1, 8, 64), "bf16"), "bf16", device)
    bt = torch.tensor(tables, dtype=torch.int32, device=device)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    before = storage.clone()
    out = A.flash_attn_with_kvcache(q, view[0, 0], view[0, 1], k=key, v=val,
                                    cache_seqlens=torch.from_numpy(ctx.astype(np.int32)).to(device),
                                    block_table=bt)
    torch.cuda.synchronize()
    kb = to_bits(before[:, 0, 0])
    vb = to_bits(before[:, 0, 1])
    with_room = [1, 2]
    slots = ko.slot_mapping([tables[b] for b in with_room], ctx[with_room], ctx[with_room] + 1)
    ko.reshape_and_cache_flash(to_bits(key)[with_room, 0], to_bits(val)[with_room, 0], kb, vb,
                               slots)
    assert np.array_equal(to_bits(storage[:, 0, 0]), kb)
    assert np.array_equal(to_bits(storage[:, 0, 1]), vb)
    ref = ko.paged_decode_attention(ko.bits_to_float(to_bits(q)[:, 0], "bf16"),
                                    ko.bits_to_float(kb, "bf16"), ko.bits_to_float(vb, "bf16"),
                                    np.asarray(tables), np.minimum(ctx + 1, 32), 1 / math.sqrt(64))
    _check(to_bits(out).reshape(3, 8, 64), ref, "bf16")


def test_fused_append_batch_above_one_launch(device):
    """2500 sequences (two launches of the unplanned kernel, several rows of
    cache copies in the merge kernel): output and cache equal the two-launch
    pattern's."""
    rng = np.random.default_rng(51)
    lens = rng.integers(1, 90, 2500)
    lens, tables, storage, key, val, q, bt, sl, slots = _fused_case(device, lens, 1, 16, 8, 64,
                                                                    "bf16", 52)
    ml = int(lens.max())
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[0, 0], view2[0, 1], slots)
    ref = A.paged_decode_attention(q, view2[0, 0], view2[0, 1], bt, sl, 0.125, ml)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    got = A.paged_decode_attention(q, view[0, 0], view[0, 1], bt, sl, 0.125, ml, key=key,
                                   value=val)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))


def _sampled_oracle(q, kc, vc, tables, lens, sel, scale, dtype):
    """The float64 oracle for sequences `sel` only, over a cache cut down to
    their blocks (tables renumbered into it)."""
    need = sorted({int(x) for b in sel for x in tables[b][:-(-int(lens[b]) // 16)]})
    where = {x: i for i, x in enumerate(need)}
    idx = torch.tensor(need, dtype=torch.int64, device=kc.device)
    k_small = to_bits(kc.index_select(0, idx))
    v_small = to_bits(vc.index_select(0, idx))
    sub = ko.pad_block_tables([[where[int(x)] for x in tables[b][:-(-int(lens[b]) // 16)]]
                               for b in sel])
    return ko.paged_decode_attention(ko.bits_to_float(to_bits(q)[sel], dtype),
                                     ko.bits_to_float(k_small, dtype),
                                     ko.bits_to_float(v_small, dtype), sub, lens[sel], scale)


def test_fused_append_qwen_full_batch(device):
    """The Qwen2.5-7B decode batch (128 sequences up to 8192 tokens), planned,
    in the 28-layer storage: the fused call equals the two-launch pattern for
    every layer of a step that shares one plan, and on sampled sequences (the
    longest, the shortest and six more) it is within the float64 oracle's
    tolerance."""
    wb = qwen_attention_batch(0)
    g = wb.geometry
    gen = torch.Generator(device=device).manual_seed(53)
    N = wb.n_pool_blocks
    storage = torch.empty((N, 4, 2, 16, g.n_kv_heads, g.head_dim), dtype=torch.bfloat16,
                          device=device)
    storage.normal_(generator=gen)
    two = storage.clone()
    bt = torch.from_numpy(wb.padded_tables()).to(device)
    sl = torch.from_numpy(wb.seq_lens.astype(np.int32)).to(device)
    slots = torch.from_numpy(wb.slot_mapping()).to(device)
    ml = int(wb.seq_lens.max())
    plan = A.DecodePlan(bt, sl, ml, g.n_kv_heads)
    view, view2 = storage.permute(1, 2, 0, 3, 4, 5), two.permute(1, 2, 0, 3, 4, 5)
    lens = wb.seq_lens.astype(np.int64)
    order = np.argsort(lens)
    rng = np.random.default_rng(53)
    sel = np.unique(np.concatenate([order[:1], order[-1:],
                                    rng.choice(wb.batch, 6, replace=False)]))
    for layer in range(4):
        q = torch.randn((wb.batch, 28, 128), generator=gen, device=device).to(torch.bfloat16)
        k = torch.randn((wb.batch, 4, 128), generator=gen, device=device).to(torch.bfloat16)
        v = torch.randn((wb.batch, 4, 128), generator=gen, device=device).to(torch.bfloat16)
        A.reshape_and_cache_flash(k, v, view2[layer, 0], view2[layer, 1], slots)
        ref = A.paged_decode_attention(q, view2[layer, 0], view2[layer, 1], None, None,
                                       1 / math.sqrt(128), ml, plan=plan)
        got = A.paged_decode_attention(q, view[layer, 0], view[layer, 1], None, None,
                                       1 / math.sqrt(128), ml, plan=plan, key=k, value=v)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), layer
        oracle = _sampled_oracle(q, view2[layer, 0], view2[layer, 1], wb.block_tables, lens,
                                 sel, 1 / math.sqrt(128), "bf16")
        _check(to_bits(got)[sel], oracle, "bf16")
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))


def test_flash_attn_with_kvcache_appends(device):
    """flash-attn's kvcache semantics: k/v land at position cache_seqlens[b]
    and the attention covers cache_seqlens[b] + 1 tokens."""
    rng = np.random.default_rng(54)
    ctx = np.asarray([0, 15, 16, 70], dtype=np.int64)
    lens, tables, storage, key, val, q, bt, sl, slots = _fused_case(device, ctx + 1, 1, 8, 2, 64,
                                                                    "bf16", 55)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    before = storage.clone()
    out = A.flash_attn_with_kvcache(q.view(4, 1, 8, 64), view[0, 0], view[0, 1],
                                    k=key.view(4, 1, 2, 64), v=val.view(4, 1, 2, 64),
                                    cache_seqlens=torch.from_numpy(ctx.astype(np.int32)).to(device),
                                    block_table=bt)
    torch.cuda.synchronize()
    kb = to_bits(before[:, 0, 0])
    vb = to_bits(before[:, 0, 1])
    ko.reshape_and_cache_flash(to_bits(key), to_bits(val), kb, vb, slots.cpu().numpy())
    assert np.array_equal(to_bits(storage[:, 0, 0]), kb)
    assert np.array_equal(to_bits(storage[:, 0, 1]), vb)
    ref = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), "bf16"),
                                    ko.bits_to_float(kb, "bf16"), ko.bits_to_float(vb, "bf16"),
                                    ko.pad_block_tables(tables), ctx + 1, 1 / math.sqrt(64))
    _check(to_bits(out).reshape(4, 8, 64), ref, "bf16")


def test_one_long_sequence_among_short_ones(device):
    """A 131072-token sequence (8192 blocks) beside short ones and an empty
    one.  The default grid cuts it into a piece per workgroup; 8192
    workgroups (the most a call takes) cut it into pieces of about one block,
    which the combine merges over hundreds of load rounds.  For both grids the
    planned call equals the unplanned one bit for bit and the output is within
    the float64 oracle's tolerance.  The appending call over the same tables
    equals the two-launch pattern and leaves the same cache."""
    Hq, Hkv, D = 28, 4, 128
    lens = np.asarray([131072, 1, 17, 5000, 0], dtype=np.int64)
    rng = np.random.default_rng(71)
    need = [-(-int(x) // 16) for x in lens]
    N = sum(need) + 8
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    gen = torch.Generator(device=device).manual_seed(71)
    storage = torch.empty((N, 1, 2, 16, Hkv, D), dtype=torch.bfloat16, device=device)
    storage.normal_(generator=gen)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    kc, vc = view[0, 0], view[0, 1]
    q = torch.randn((len(lens), Hq, D), generator=gen, device=device).to(torch.bfloat16)
    bt = torch.from_numpy(padded).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    ml = int(lens.max())
    scale = 1.0 / math.sqrt(D)
    oracle = ko.paged_decode_attention(ko.bits_to_float(to_bits(q), "bf16"),
                                       ko.bits_to_float(to_bits(kc), "bf16"),
                                       ko.bits_to_float(to_bits(vc), "bf16"), padded, lens, scale)
    for nwg in (0, 8192):
        ref = A.paged_decode_attention(q, kc, vc, bt, sl, scale, ml, n_workgroups=nwg)
        plan = A.DecodePlan(bt, sl, ml, Hkv, nwg)
        got = A.paged_decode_attention(q, kc, vc, None, None, scale, ml, n_workgroups=nwg,
                                       plan=plan)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), nwg
        _check(to_bits(got), oracle, "bf16")

    # the same tables with a new token at the end of each non-empty sequence
    n = 4
    key = torch.randn((n, Hkv, D), generator=gen, device=device).to(torch.bfloat16)
    val = torch.randn((n, Hkv, D), generator=gen, device=device).to(torch.bfloat16)
    slots = torch.from_numpy(ko.slot_mapping(tables[:n], lens[:n] - 1, lens[:n])).to(device)
    two = storage.clone()
    view2 = two.permute(1, 2, 0, 3, 4, 5)
    A.reshape_and_cache_flash(key, val, view2[0, 0], view2[0, 1], slots)
    ref = A.paged_decode_attention(q[:n], view2[0, 0], view2[0, 1], bt[:n], sl[:n], scale, ml)
    got = A.paged_decode_attention(q[:n], kc, vc, bt[:n], sl[:n], scale, ml, key=key, value=val)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))


def test_flash_attn_with_kvcache_reuses_the_step_plan(device):
    """The vLLM-facing call plans once per step: the layers of a step, which
    pass the same block_table and cache_seqlens tensors, reuse the plan built
    at the first (bit-identical to unplanned calls); an in-place edit of the
    lengths, new tensors with the same contents, or an appending call build a
    new one."""
    rng = np.random.default_rng(81)
    ctx = np.asarray([0, 15, 16, 70, 300, 1], dtype=np.int64)
    lens, tables, storage, key, val, q, bt, sl, slots = _fused_case(device, ctx + 1, 2, 8, 2, 64,
                                                                    "bf16", 82)
    view = storage.permute(1, 2, 0, 3, 4, 5)
    kc, vc = view[0, 0], view[0, 1]
    cs = torch.from_numpy(ctx.astype(np.int32)).to(device)
    q4 = q.view(len(ctx), 1, 8, 64)
    ms = bt.size(1) * 16

    def unplanned(lengths):
        return A.paged_decode_attention(q, kc, vc, bt, lengths, 1 / math.sqrt(64), ms)

    out1 = A.flash_attn_with_kvcache(q4, kc, vc, cache_seqlens=cs, block_table=bt)
    plan1 = A._step_plans._by_device[q.device.index][3]
    out2 = A.flash_attn_with_kvcache(q4, kc, vc, cache_seqlens=cs, block_table=bt)
    assert A._step_plans._by_device[q.device.index][3] is plan1 and plan1 is not None
    ref = unplanned(cs)
    torch.cuda.synchronize()
    assert torch.equal(out1.view(torch.int16), out2.view(torch.int16))
    assert torch.equal(out1.view(-1).view(torch.int16), ref.view(-1).view(torch.int16))

    cs[4] -= 100  # an in-place edit of the step's lengths
    out3 = A.flash_attn_with_kvcache(q4, kc, vc, cache_seqlens=cs, block_table=bt)
    assert A._step_plans._by_device[q.device.index][3] is not plan1
    ref3 = unplanned(cs)
    torch.cuda.synchronize()
    assert torch.equal(out3.view(-1).view(torch.int16), ref3.view(-1).view(torch.int16))

    plan3 = A._step_plans._by_device[q.device.index][3]
    cs2 = cs.clone()  # the next step's tensors, same contents
    A.flash_attn_with_kvcache(q4, kc, vc, cache_seqlens=cs2, block_table=bt)
    assert A._step_plans._by_device[q.device.index][3] is not plan3

    # appending: the plan counts the new token; cache and output as the
    # unplanned appending call leaves them
    two = storage.clone()
    v2 = two.permute(1, 2, 0, 3, 4, 5)
    k4, vv4 = key.view(len(ctx), 1, 2, 64), val.view(len(ctx), 1, 2, 64)
    got = A.flash_attn_with_kvcache(q4, kc, vc, k=k4, v=vv4, cache_seqlens=cs2, block_table=bt)
    ref_app = A.paged_decode_attention(q, v2[0, 0], v2[0, 1], bt, cs2 + 1, 1 / math.sqrt(64), ms,
                                       key=key, value=val)
    torch.cuda.synchronize()
    assert torch.equal(storage.view(torch.int16), two.view(torch.int16))
    assert torch.equal(got.view(-1).view(torch.int16), ref_app.view(-1).view(torch.int16))
