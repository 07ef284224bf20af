"""Pins of the CPU oracle (runs without a GPU).

Each check fixes an oracle function by something other than the oracle's own
formula: the golden fixture written by per-element flat-index loops
(tests/golden/make_golden.py), hand-computed literals, torch's float64
scaled_dot_product_attention, closed forms of softmax attention, torch's own
bf16/fp16 rounding, and brute force on tiny inputs.  A plausible slip in the
oracle (a transposed view, h % G instead of h // G for GQA, an off-by-one in
the slot formula, a dropped max-subtraction) fails at least one of them.
"""
import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as ko
from tests.kvtest_utils import load_golden, random_bits


# ---------------------------------------------------------------- golden fixture
def test_golden_slots_match_oracle_slot_mapping():
    z = load_golden()
    ctx = z["context_lens"]
    nb = [-(-int(c + 1) // 16) for c in ctx]
    tables = [list(map(int, z["tables"][i, :nb[i]])) for i in range(len(ctx))]
    got = ko.slot_mapping(tables, ctx, ctx + 1)
    assert np.array_equal(got, z["slots"])


def test_golden_append_matches_oracle():
    z = load_golden()
    N, L, H, D, BS = (int(x) for x in z["geometry"])
    pool = z["pool"].copy().reshape(N, L, 2, BS, H, D)
    ko.append_layers(z["new_k"].reshape(1, -1, H, D), z["new_v"].reshape(1, -1, H, D), pool,
                     z["slots"])
    expect = z["pool"].copy()
    expect[z["append_idx"]] = z["append_val"]
    assert np.array_equal(pool.reshape(-1), expect)


def test_golden_gather_matches_oracle():
    z = load_golden()
    N, L, H, D, BS = (int(x) for x in z["geometry"])
    pool = z["pool"].copy()
    pool[z["append_idx"]] = z["append_val"]
    sl = z["seq_lens"]
    tables = [list(map(int, z["tables"][i, :-(-int(ln) // BS)])) for i, ln in enumerate(sl)]
    ok_, ov = ko.gather_tokens(pool.reshape(N, L, 2, BS, H, D), tables, sl)
    assert np.array_equal(ok_[0], z["out_k"])
    assert np.array_equal(ov[0], z["out_v"])


def test_golden_swap_matches_oracle():
    z = load_golden()
    N, L, H, D, BS = (int(x) for x in z["geometry"])
    pool = z["pool"].copy()
    pool[z["append_idx"]] = z["append_val"]
    n = len(z["swap_src"])
    host = np.zeros((n, L, 2, BS, H, D), dtype=np.uint16)
    ko.swap_blocks(z["swap_src"], z["swap_dst"], False, pool.reshape(N, L, 2, BS, H, D), host)
    assert np.array_equal(host.reshape(-1), z["host_after_swap"])


# ---------------------------------------------------------------- literals
def test_slot_mapping_literals():
    bt = [[7, 3, 9]]
    # positions 0, 15, 16, 17, 33 of one sequence (context 0, seq_len 34)
    got = ko.slot_mapping(bt, [0], [34])
    assert got[0] == 112 and got[15] == 127 and got[16] == 48 and got[17] == 49
    assert got[32] == 144 and got[33] == 145
    # only the new tokens [context_len, seq_len) are mapped, concatenated over requests
    got = ko.slot_mapping([[5], [2, 8]], [15, 16], [16, 18])
    assert got.tolist() == [95, 128, 129]
    assert ko.slot_mapping([[4]], [0], [1]).tolist() == [64]  # length 1


def test_pad_block_tables_literal():
    out = ko.pad_block_tables([[3, 1], [], [9, 8, 7]])
    assert out.dtype == np.int32
    assert out.tolist() == [[3, 1, 0], [0, 0, 0], [9, 8, 7]]


def test_append_literal_index():
    """storage [N, L, 2, 16, H, D]: layer l's key row of slot s sits at
    flat ((((s//16)*L + l)*2 + 0)*16 + s%16)*H*D."""
    N, L, H, D = 5, 3, 2, 4
    st = np.zeros((N, L, 2, 16, H, D), dtype=np.int64)
    key = np.arange(L * 2 * H * D).reshape(L, 2, H, D) + 1
    val = -key
    ko.append_layers(key, val, st, np.asarray([37, -1]))
    flat = st.reshape(-1)
    for l in range(L):
        kb = ((((37 // 16) * L + l) * 2 + 0) * 16 + 37 % 16) * H * D
        vb = ((((37 // 16) * L + l) * 2 + 1) * 16 + 37 % 16) * H * D
        assert np.array_equal(flat[kb:kb + H * D], key[l, 0].reshape(-1))
        assert np.array_equal(flat[vb:vb + H * D], val[l, 0].reshape(-1))
    assert np.count_nonzero(flat) == 2 * L * H * D  # slot -1 wrote nothing


def test_brute_force_pack_scatter_copy():
    rng = np.random.default_rng(0)
    pool = rng.integers(0, 256, size=(9, 24), dtype=np.uint8)
    ids = [4, 0, 7]
    st = ko.pack_blocks(pool, ids)
    for i, b in enumerate(ids):
        for j in range(24):
            assert st[i, j] == pool[b, j]
    other = np.zeros_like(pool)
    ko.scatter_blocks(st, [8, 1, 2], other)
    assert np.array_equal(other[[8, 1, 2]], pool[ids]) and not other[[0, 3, 4, 5, 6, 7]].any()
    third = np.zeros_like(pool)
    ko.copy_blocks(pool, third, None, [5, 6])
    assert np.array_equal(third[5], pool[0]) and np.array_equal(third[6], pool[1])


def test_swap_later_pair_wins_on_duplicate_destination():
    """The reference issues its copies in list order on one stream
    (aegaeon/ops/swap.cu:36-58), so a repeated destination keeps the last."""
    cache = np.arange(4 * 2).reshape(4, 2).astype(np.uint16)
    host = np.zeros((2, 2), dtype=np.uint16)
    ko.swap_blocks([1, 3], [0, 0], False, cache, host)
    assert host[0].tolist() == cache[3].tolist()


# ---------------------------------------------------------------- dtype rounding
@pytest.mark.parametrize("dtype,tdt", [("bf16", torch.bfloat16), ("fp16", torch.float16)])
def test_bit_conversions_match_torch(dtype, tdt):
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(4000) * 10.0 ** rng.integers(-6, 5, 4000),
                        [0.0, -0.0, 1.0, 65504.0, 1e-8, np.inf, -np.inf]]).astype(np.float32)
    got = ko.float_to_bits(x, dtype)
    want = torch.from_numpy(x).to(tdt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    back = ko.bits_to_float(want, dtype)
    assert np.array_equal(back, torch.from_numpy(want.view(np.int16)).view(tdt).double().numpy())


# ---------------------------------------------------------------- attention
def _paged_case(rng, lens, Hq, Hkv, D, dtype="bf16"):
    need = [-(-int(x) // 16) for x in lens]
    N = 2 * sum(need) + 3
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    kc = ko.bits_to_float(random_bits(rng, (N, 16, Hkv, D), dtype), dtype)
    vc = ko.bits_to_float(random_bits(rng, (N, 16, Hkv, D), dtype), dtype)
    q = ko.bits_to_float(random_bits(rng, (len(lens), Hq, D), dtype), dtype)
    return tables, ko.pad_block_tables(tables), q, kc, vc


@pytest.mark.parametrize("Hq,Hkv,D", [(28, 4, 128), (8, 8, 64), (6, 2, 32)])
def test_attention_matches_torch_sdpa_fp64(Hq, Hkv, D):
    rng = np.random.default_rng(Hq + D)
    lens = [1, 16, 17, 40]
    tables, padded, q, kc, vc = _paged_case(rng, lens, Hq, Hkv, D)
    scale = 1 / math.sqrt(D)
    got = ko.paged_decode_attention(q, kc, vc, padded, lens, scale)
    G = Hq // Hkv
    for b, ln in enumerate(lens):
        # gather the sequence by explicit per-token block lookups
        k = np.stack([kc[tables[b][p // 16], p % 16] for p in range(ln)])  # [T, Hkv, D]
        v = np.stack([vc[tables[b][p // 16], p % 16] for p in range(ln)])
        kt = torch.from_numpy(k).permute(1, 0, 2).repeat_interleave(G, dim=0)  # [Hq, T, D]
        vt = torch.from_numpy(v).permute(1, 0, 2).repeat_interleave(G, dim=0)
        qt = torch.from_numpy(q[b]).unsqueeze(1)  # [Hq, 1, D]
        want = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, scale=scale)
        np.testing.assert_allclose(got[b], want[:, 0].numpy(), rtol=1e-12, atol=1e-12)


def test_attention_closed_forms():
    rng = np.random.default_rng(3)
    Hq, Hkv, D = 8, 2, 16
    tables, padded, q, kc, vc = _paged_case(rng, [1, 30], Hq, Hkv, D)
    # len 1: output is V0 of each sequence's kv head, for every query head of the group
    out = ko.paged_decode_attention(q, kc, vc, padded, [1, 30], 0.125)
    assert np.array_equal(out[0], np.repeat(vc[tables[0][0], 0], Hq // Hkv, axis=0))
    # equal keys: uniform softmax -> mean of the values
    kc2 = kc.copy()
    kc2[:] = kc[0, 0]
    out = ko.paged_decode_attention(q, kc2, vc, padded, [1, 30], 0.125)
    v = np.stack([vc[tables[1][p // 16], p % 16] for p in range(30)]).mean(axis=0)
    np.testing.assert_allclose(out[1], np.repeat(v, Hq // Hkv, axis=0), rtol=1e-12, atol=1e-12)
    # a dominant logit selects its value row; large logits must not overflow
    kc3 = kc.copy() * 0.0
    kc3[tables[1][1], 3] = 1000.0  # token 19
    q3 = np.abs(q) + 1.0
    out = ko.paged_decode_attention(q3, kc3, vc, padded, [1, 30], 1.0)
    assert np.isfinite(out).all()
    np.testing.assert_allclose(out[1], np.repeat(vc[tables[1][1], 3], Hq // Hkv, axis=0),
                               rtol=0, atol=1e-9)


def test_attention_gqa_equals_mha_with_repeated_heads():
    rng = np.random.default_rng(4)
    tables, padded, q, kc, vc = _paged_case(rng, [23, 5], 6, 2, 32)
    gqa = ko.paged_decode_attention(q, kc, vc, padded, [23, 5], 0.2)
    mha = ko.paged_decode_attention(q, np.repeat(kc, 3, axis=2), np.repeat(vc, 3, axis=2),
                                    padded, [23, 5], 0.2)
    np.testing.assert_allclose(gqa, mha, rtol=1e-12, atol=1e-12)


def test_attention_ignores_padding_and_stale_rows():
    rng = np.random.default_rng(5)
    tables, padded, q, kc, vc = _paged_case(rng, [5, 18], 4, 2, 16)
    ref = ko.paged_decode_attention(q, kc, vc, padded, [5, 18], 0.25)
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[tables[0][0], 5:] = np.nan
    vc2[tables[1][1], 2:] = np.nan
    wide = np.pad(padded, ((0, 0), (0, 3)))
    out = ko.paged_decode_attention(q, kc2, vc2, wide, [5, 18], 0.25)
    assert np.array_equal(out, ref)


# ---------------------------------------------------------------- defrag plan
@pytest.mark.parametrize("seed", range(5))
def test_defrag_plan_invariants(seed):
    rng = np.random.default_rng(seed)
    valid = sorted(rng.permutation(400)[:150].tolist())  # a shape's (sparse) id space
    live = rng.permutation(valid)[:70].tolist()
    src, dst = ko.plan_defrag(live, valid)
    assert not set(src) & set(dst)
    assert len(set(src)) == len(src) == len(set(dst)) == len(dst)
    tables = [live[i:i + 7] for i in range(0, 70, 7)]
    new = ko.apply_defrag(tables, src, dst)
    assert sorted(x for t in new for x in t) == valid[:70]  # dense prefix of the id space
    # brute force: byte payloads follow their blocks
    pool = {b: rng.integers(0, 1 << 30) for b in valid}
    moved = dict(pool)
    for s, d in zip(src, dst):
        moved[d] = pool[s]
    for old, nw in zip(tables, new):
        assert [pool[x] for x in old] == [moved[x] for x in nw]
    # already-dense pools move nothing
    assert ko.plan_defrag(valid[:30], valid) == ([], [])


def test_prepare_model_inputs_literal():
    """worker.py:596-676 on a prefill + two decodes, values worked by hand:
    slot = table[p // 16] * 16 + p % 16; prefill rows of the padded table
    are empty; start offsets are prefix sums."""
    reqs = [(0, [11, 12, 13], 3, 0), (1, [7], 18, 17), (2, [9], 33, 32)]
    r = ko.prepare_model_inputs(reqs, [[5], [2, 9], [4, 6, 8]])
    assert r["slot_mapping"].tolist() == [80, 81, 82, 9 * 16 + 1, 8 * 16]
    assert r["input_positions"].tolist() == [0, 1, 2, 17, 32]
    assert r["input_tokens"].tolist() == [11, 12, 13, 7, 9]
    assert r["block_tables"].tolist() == [[0, 0, 0], [2, 9, 0], [4, 6, 8]]
    assert r["block_tables"].dtype == np.int32 and r["slot_mapping"].dtype == np.int64
    assert r["query_start_loc"].tolist() == [0, 3, 4, 5]
    assert r["seq_start_loc"].tolist() == [0, 3, 21, 54]
    assert (r["num_prefills"], r["num_prefill_tokens"], r["num_decode_tokens"]) == (1, 3, 2)
    assert (r["max_query_len"], r["max_prefill_seq_len"], r["max_decode_seq_len"]) == (3, 3, 33)


# ---------------------------------------------------------------------------
# varlen prefill attention
# ---------------------------------------------------------------------------
def _packed_case(rng, lens, Hq, Hkv, D):
    cu = np.concatenate([[0], np.cumsum(lens)]).astype(np.int64)
    T = int(cu[-1])
    q = rng.standard_normal((T, Hq, D))
    k = rng.standard_normal((T, Hkv, D))
    v = rng.standard_normal((T, Hkv, D))
    return cu, q, k, v


@pytest.mark.parametrize("Hq,Hkv,D", [(4, 4, 16), (6, 2, 32), (7, 1, 8)])
@pytest.mark.parametrize("causal", [True, False])
def test_prefill_matches_torch_sdpa_fp64(Hq, Hkv, D, causal):
    """torch's own causal SDPA in float64, one sequence at a time, with the
    kv heads repeated for GQA (head h reads kv head h // G)."""
    rng = np.random.default_rng(Hq * 10 + D)
    lens = [1, 5, 17, 33]
    cu, q, k, v = _packed_case(rng, lens, Hq, Hkv, D)
    scale = 0.3
    got = ko.varlen_prefill_attention(q, k, v, cu, scale, causal)
    G = Hq // Hkv
    for b in range(len(lens)):
        s0, s1 = cu[b], cu[b + 1]
        qt = torch.from_numpy(q[s0:s1]).transpose(0, 1)               # [Hq, n, D]
        kt = torch.from_numpy(k[s0:s1]).transpose(0, 1).repeat_interleave(G, 0)
        vt = torch.from_numpy(v[s0:s1]).transpose(0, 1).repeat_interleave(G, 0)
        want = torch.nn.functional.scaled_dot_product_attention(
            qt.contiguous(), kt.contiguous(), vt.contiguous(), scale=scale, is_causal=causal)
        np.testing.assert_allclose(got[s0:s1], want.transpose(0, 1).numpy(), rtol=1e-12,
                                   atol=1e-12)


def test_prefill_closed_forms():
    """Causal: query 0 sees only key 0, so its output is v[0]; with equal keys
    query i outputs the mean of v[0..i]; a dominant logit picks its value row."""
    rng = np.random.default_rng(9)
    cu, q, k, v = _packed_case(rng, [6, 9], 4, 2, 8)
    out = ko.varlen_prefill_attention(q, k, v, cu, 0.5, True)
    for b in range(2):
        s0 = cu[b]
        np.testing.assert_allclose(out[s0], np.repeat(v[s0], 2, axis=0), rtol=1e-14)
    k_eq = np.broadcast_to(k[:1], k.shape).copy()
    out = ko.varlen_prefill_attention(q, k_eq, v, cu, 0.5, True)
    for b in range(2):
        s0, s1 = cu[b], cu[b + 1]
        for i in range(s1 - s0):
            want = np.repeat(v[s0:s0 + i + 1].mean(axis=0), 2, axis=0)
            np.testing.assert_allclose(out[s0 + i], want, rtol=1e-12, atol=1e-12)
    out = ko.varlen_prefill_attention(q, k_eq, v, cu, 0.5, False)
    np.testing.assert_allclose(out[cu[1] + 2], np.repeat(v[cu[1]:].mean(axis=0), 2, axis=0),
                               rtol=1e-12, atol=1e-12)
    k_dom = k.copy()
    q1 = np.zeros_like(q)
    q1[:, :, 0] = 1.0
    k_dom[:, :, 0] = 0.0
    k_dom[cu[1] + 3, :, 0] = 500.0                     # key 3 of sequence 1
    out = ko.varlen_prefill_attention(q1, k_dom, v, cu, 1.0, True)
    np.testing.assert_allclose(out[cu[1] + 7], np.repeat(v[cu[1] + 3], 2, axis=0), rtol=1e-12)
    np.testing.assert_allclose(out[cu[1] + 2], np.repeat(v[cu[1]:cu[1] + 3].mean(axis=0), 2,
                                                         axis=0), rtol=1e-12)


def test_prefill_gqa_equals_mha_with_repeated_heads():
    rng = np.random.default_rng(10)
    cu, q, k, v = _packed_case(rng, [12, 3, 20], 6, 2, 16)
    gqa = ko.varlen_prefill_attention(q, k, v, cu, 0.2, True)
    mha = ko.varlen_prefill_attention(q, np.repeat(k, 3, axis=1), np.repeat(v, 3, axis=1), cu,
                                      0.2, True)
    np.testing.assert_allclose(gqa, mha, rtol=1e-12, atol=1e-14)


from hypothesis import given, settings, strategies as st  # noqa: E402


@settings(max_examples=60, deadline=None)
@given(data=st.data())
def test_oracle_swap_matches_per_byte_loop(data):
    """The oracle's swap against an explicit per-byte copy on random pools and
    id lists, in both directions, repeated destinations included (the last
    write wins, swap.cu:36-58 copies in order)."""
    n_dev = data.draw(st.integers(1, 12))
    n_host = data.draw(st.integers(1, 12))
    bb = data.draw(st.sampled_from([2, 6, 32]))
    n = data.draw(st.integers(0, 10))
    swap_in = data.draw(st.booleans())
    src_n, dst_n = (n_host, n_dev) if swap_in else (n_dev, n_host)
    src = data.draw(st.lists(st.integers(0, src_n - 1), min_size=n, max_size=n))
    dst = data.draw(st.lists(st.integers(0, dst_n - 1), min_size=n, max_size=n))
    rng = np.random.default_rng(data.draw(st.integers(0, 1000)))
    dev = rng.integers(0, 256, (n_dev, bb), dtype=np.uint8)
    host = rng.integers(0, 256, (n_host, bb), dtype=np.uint8)
    want_dev, want_host = dev.copy(), host.copy()
    s_pool, d_pool = (want_host, want_dev) if swap_in else (want_dev, want_host)
    for i in range(n):
        for byte in range(bb):
            d_pool[dst[i], byte] = s_pool[src[i], byte]
    ko.swap_blocks(src, dst, swap_in, dev, host)
    assert np.array_equal(dev, want_dev) and np.array_equal(host, want_host)


# ---------------------------------------------------------------------------
# the torch CPU restatement (the timed CPU baseline) against the numpy oracle
# ---------------------------------------------------------------------------
def _bits_tensor(bits, dtype):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(dtype)


def test_torch_cpu_append_matches_oracle():
    """Bit-exact against ko.append_layers, slot -1 skipped, blocks of other
    sequences untouched (both start from the same poisoned pool)."""
    from oracle import torch_cpu as tc
    rng = np.random.default_rng(61)
    N, L, H, D = 20, 3, 2, 64
    pool = random_bits(rng, (N, L, 2, 16, H, D), "bf16")
    key = random_bits(rng, (L, 9, H, D), "bf16")
    val = random_bits(rng, (L, 9, H, D), "bf16")
    slots = np.asarray([5, 17, 16, -1, 300, 31, 2, 319, 64], dtype=np.int64)
    ref = pool.copy()
    ko.append_layers(key, val, ref, slots)
    got = _bits_tensor(pool.copy(), torch.bfloat16)
    tc.append_layers(_bits_tensor(key, torch.bfloat16), _bits_tensor(val, torch.bfloat16), got,
                     torch.from_numpy(slots))
    assert np.array_equal(got.view(torch.int16).numpy().view(np.uint16), ref)


def test_torch_cpu_attention_matches_oracle():
    """float32 from 16-bit inputs within 1e-5 relative L2 of the float64
    oracle (GQA 7, ragged lengths, a zero length, scattered tables)."""
    from oracle import torch_cpu as tc
    rng = np.random.default_rng(62)
    lens = [1, 15, 16, 17, 0, 130]
    need = [-(-x // 16) for x in lens]
    N = 2 * sum(need) + 3
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    q = random_bits(rng, (len(lens), 14, 64), "bf16")
    kc = random_bits(rng, (N, 16, 2, 64), "bf16")
    vc = random_bits(rng, (N, 16, 2, 64), "bf16")
    ref = ko.paged_decode_attention(ko.bits_to_float(q, "bf16"), ko.bits_to_float(kc, "bf16"),
                                    ko.bits_to_float(vc, "bf16"), padded, lens, 0.125)
    got = tc.paged_decode_attention(_bits_tensor(q, torch.bfloat16),
                                    _bits_tensor(kc, torch.bfloat16),
                                    _bits_tensor(vc, torch.bfloat16), torch.from_numpy(padded),
                                    torch.tensor(lens), 0.125).double().numpy()
    assert np.linalg.norm(got - ref) / np.linalg.norm(ref) < 1e-5
    assert not got[4].any()


def test_torch_cpu_swap_matches_oracle():
    from oracle import torch_cpu as tc
    rng = np.random.default_rng(63)
    gpu = random_bits(rng, (12, 2, 16, 1, 64), "fp16")
    host = np.zeros((6, 2, 16, 1, 64), dtype=np.uint16)
    src, dst = [7, 2, 11, 2], [0, 5, 3, 1]
    ref = host.copy()
    ko.swap_blocks(src, dst, False, gpu.copy(), ref)
    got = torch.from_numpy(host.copy().view(np.int16))
    tc.swap_blocks(src, dst, torch.from_numpy(gpu.view(np.int16)), got)
    assert np.array_equal(got.numpy().view(np.uint16), ref)
