"""GPU parity of the slot-mapped append (vLLM reshape_and_cache_flash semantics,
reached from aegaeon/aegaeon/worker.py:517-523) and the block-table gather."""
import numpy as np
import pytest
import torch

from aegaeon_amd import attention as A
from aegaeon_amd.workloads import QWEN25_7B, qwen_append_batch
from oracle import kv_oracle as ko
from tests.kvtest_utils import load_golden, random_bits, to_bits, to_device_bits

pytestmark = pytest.mark.gpu


def test_golden_append_then_gather(device):
    z = load_golden()
    N, L, H, D, BS = (int(x) for x in z["geometry"])
    cache = to_device_bits(z["pool"], "fp16", device).view(N, L, 2, BS, H, D)
    key = to_device_bits(z["new_k"], "fp16", device).view(1, -1, H, D)
    val = to_device_bits(z["new_v"], "fp16", device).view(1, -1, H, D)
    slots = torch.from_numpy(z["slots"]).to(device)
    A.append_kv(key, val, cache, slots)
    expect = z["pool"].copy()
    expect[z["append_idx"]] = z["append_val"]
    assert np.array_equal(to_bits(cache).reshape(-1), expect)
    sl = z["seq_lens"]
    bt = torch.from_numpy(z["tables"]).to(device)
    out_k, out_v = A.gather_tokens(cache, bt, torch.from_numpy(sl.astype(np.int32)).to(device),
                                   int(sl.sum()), int(sl.max()))
    assert np.array_equal(to_bits(out_k)[0], z["out_k"])
    assert np.array_equal(to_bits(out_v)[0], z["out_v"])


def test_per_layer_reshape_and_cache_flash(device):
    """vLLM's per-layer call through the permuted view (worker.py:419-451)
    equals the oracle, including padding slots (-1) and strided keys."""
    rng = np.random.default_rng(11)
    N, L, H, D = 40, 3, 4, 128
    bits = random_bits(rng, (N, L, 2, 16, H, D), "bf16")
    cache = to_device_bits(bits, "bf16", device)
    view = cache.permute(1, 2, 0, 3, 4, 5)
    T = 37
    qkv = to_device_bits(random_bits(rng, (T, 3 * H * D), "bf16"), "bf16", device)
    key = qkv[:, H * D:2 * H * D].view(T, H, D)      # token stride 3*H*D
    val = qkv[:, 2 * H * D:].view(T, H, D)
    slots_np = rng.permutation(N * 16)[:T].astype(np.int64)
    slots_np[[3, 20]] = -1
    slots = torch.from_numpy(slots_np).to(device)
    ref = bits.copy()
    rview = ref.transpose(1, 2, 0, 3, 4, 5)
    kb, vb = to_bits(key), to_bits(val)
    for layer in range(L):
        A.reshape_and_cache_flash(key, val, view[layer, 0], view[layer, 1], slots)
        ko.reshape_and_cache_flash(kb, vb, rview[layer, 0], rview[layer, 1], slots_np)
    assert np.array_equal(to_bits(cache), ref)


def test_out_of_range_slots_skipped(device):
    """Slots < 0 and >= N*16 never write; every other byte is untouched."""
    rng = np.random.default_rng(5)
    N, L, H, D = 8, 2, 2, 64
    cache = torch.full((N, L, 2, 16, H, D), float("nan"), dtype=torch.float16, device=device)
    before = to_bits(cache)
    key = to_device_bits(random_bits(rng, (L, 4, H, D), "fp16"), "fp16", device)
    val = to_device_bits(random_bits(rng, (L, 4, H, D), "fp16"), "fp16", device)
    slots_np = np.asarray([-1, N * 16, 5, N * 16 + 100], dtype=np.int64)
    A.append_kv(key, val, cache, torch.from_numpy(slots_np).to(device))
    got = to_bits(cache)
    ref = before.copy()
    ko.append_layers(to_bits(key), to_bits(val), ref, np.asarray([-1, -1, 5, -1]))
    assert np.array_equal(got, ref)


def test_append_rejects_short_slot_mapping(device):
    """A slot list shorter than the tokens (or not 1-d) raises before any
    launch, for both the per-layer and the all-layer call; the cache is
    untouched."""
    rng = np.random.default_rng(6)
    N, L, H, D = 8, 2, 2, 64
    cache = to_device_bits(random_bits(rng, (N, L, 2, 16, H, D), "fp16"), "fp16", device)
    before = to_bits(cache)
    key = to_device_bits(random_bits(rng, (L, 4, H, D), "fp16"), "fp16", device)
    val = to_device_bits(random_bits(rng, (L, 4, H, D), "fp16"), "fp16", device)
    view = cache.permute(1, 2, 0, 3, 4, 5)
    for slots in (torch.arange(3, dtype=torch.int64, device=device),
                  torch.arange(4, dtype=torch.int64, device=device).view(2, 2)):
        with pytest.raises(ValueError):
            A.append_kv(key, val, cache, slots)
        with pytest.raises(ValueError):
            A.reshape_and_cache_flash(key[0], val[0], view[0, 0], view[0, 1], slots)
    torch.cuda.synchronize()
    assert np.array_equal(to_bits(cache), before)


def test_qwen_full_size_append(device):
    """Qwen2.5-7B shape, 256 sequences, pool = 2x need (17.4 GB): each appended
    row reads back exactly (append -> gather identity) and no other byte
    changes (count of modified elements)."""
    wb = qwen_append_batch(0)
    g = wb.geometry
    N = wb.n_pool_blocks
    cache = torch.empty((N, *g.block_shape), dtype=torch.bfloat16, device=device)
    cache.view(torch.int16).fill_(0x7FC1)  # a NaN pattern the inputs never hold
    gen = torch.Generator(device=device).manual_seed(0)
    key = torch.randn((g.n_layers, wb.batch, g.n_kv_heads, g.head_dim), generator=gen,
                      device=device).to(torch.bfloat16)
    val = torch.randn(key.shape, generator=gen, device=device).to(torch.bfloat16)
    slots_np = wb.slot_mapping()
    slots = torch.from_numpy(slots_np).to(device)
    A.append_kv(key, val, cache, slots)
    blk = slots // 16
    off = slots % 16
    got_k = cache[blk, :, 0, off]  # [B, L, H, D]
    got_v = cache[blk, :, 1, off]
    assert torch.equal(got_k.view(torch.int16), key.transpose(0, 1).view(torch.int16))
    assert torch.equal(got_v.view(torch.int16), val.transpose(0, 1).view(torch.int16))
    changed = int((cache.view(torch.int16) != 0x7FC1).sum())
    inputs_hit_pattern = int((key.view(torch.int16) == 0x7FC1).sum() + (val.view(torch.int16) == 0x7FC1).sum())
    assert changed + inputs_hit_pattern == 2 * key.numel()


def test_gather_qwen_layers_subset(device):
    """gather of layers (5, 3) of a Qwen-shaped pool equals the oracle."""
    rng = np.random.default_rng(9)
    g = QWEN25_7B
    N = 64
    bits = random_bits(rng, (N, *g.block_shape), "bf16")
    cache = to_device_bits(bits, "bf16", device)
    lens = np.asarray([1, 15, 16, 17, 100, 0, 33], dtype=np.int64)
    need = [-(-int(x) // 16) for x in lens]
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    padded = ko.pad_block_tables(tables)
    bt = torch.from_numpy(padded).to(device)
    out_k, out_v = A.gather_tokens(cache, bt, torch.from_numpy(lens.astype(np.int32)).to(device),
                                   int(lens.sum()), int(lens.max()), layers=(5, 3))
    rk, rv = ko.gather_tokens(bits, tables, lens, layers=[5, 6, 7])
    assert np.array_equal(to_bits(out_k), rk)
    assert np.array_equal(to_bits(out_v), rv)


def _tables_for(rng, lens, N):
    need = [-(-int(x) // 16) for x in lens]
    assert sum(need) <= N
    ids = rng.permutation(N)[:sum(need)]
    tables, o = [], 0
    for c in need:
        tables.append([int(x) for x in ids[o:o + c]])
        o += c
    return tables


def test_gather_batch_above_one_launch(device):
    """2500 sequences (lengths 0..40) run as three launches of <= 1024."""
    rng = np.random.default_rng(31)
    N, L, H, D = 6000, 2, 2, 64                         # about 4500 blocks needed
    bits = random_bits(rng, (N, L, 2, 16, H, D), "fp16")
    cache = to_device_bits(bits, "fp16", device)
    lens = rng.integers(0, 41, 2500).astype(np.int64)
    tables = _tables_for(rng, lens, N)
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    out_k, out_v = A.gather_tokens(cache, bt, torch.from_numpy(lens.astype(np.int32)).to(device),
                                   int(lens.sum()), int(lens.max()))
    rk, rv = ko.gather_tokens(bits, tables, lens)
    assert np.array_equal(to_bits(out_k), rk)
    assert np.array_equal(to_bits(out_v), rv)


def test_gather_wide_rows(device):
    """Llama-2-13B rows (40 heads x 128 = 10 KiB): a 16-token block is 160 KiB,
    copied in several 16 KiB passes."""
    rng = np.random.default_rng(32)
    N, L, H, D = 24, 1, 40, 128
    bits = random_bits(rng, (N, L, 2, 16, H, D), "fp16")
    cache = to_device_bits(bits, "fp16", device)
    lens = np.asarray([16, 1, 37, 0, 95], dtype=np.int64)
    tables = _tables_for(rng, lens, N)
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    out_k, out_v = A.gather_tokens(cache, bt, torch.from_numpy(lens.astype(np.int32)).to(device),
                                   int(lens.sum()), int(lens.max()))
    rk, rv = ko.gather_tokens(bits, tables, lens)
    assert np.array_equal(to_bits(out_k), rk)
    assert np.array_equal(to_bits(out_v), rv)


def test_gather_clips_capacity_bad_ids_and_long_lengths(device):
    """Output rows past the capacity, blocks with ids outside the pool and
    tokens past the host bound max_seq_len are never written."""
    rng = np.random.default_rng(33)
    N, L, H, D = 40, 1, 2, 64
    bits = random_bits(rng, (N, L, 2, 16, H, D), "bf16")
    cache = to_device_bits(bits, "bf16", device)
    lens = np.asarray([20, 33, 50], dtype=np.int64)
    tables = _tables_for(rng, lens, N)
    tables[1][1] = N + 7                                # tokens 16..31 of sequence 1
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    max_len, cap = 40, 80                               # sequence 2 clamped to 40 tokens
    cu = torch.tensor([0, 20, 53, 93], dtype=torch.int32, device=device)
    es = cache.element_size()
    ok = torch.full((1, cap, H, D), 7.0, dtype=cache.dtype, device=device)
    ov = torch.full_like(ok, 7.0)
    from aegaeon_amd import _lib
    base = cache.data_ptr()
    rc = _lib.load().aegkv_gather_tokens(
        base, base + 16 * H * D * es, cache.stride(0), cache.stride(1), N, bt.data_ptr(),
        bt.size(1), sl.data_ptr(), cu.data_ptr(), 3, max_len, ok.data_ptr(), ov.data_ptr(), cap,
        cap * H * D, 1, 16, H, D, es, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    good = [t if i != 1 else [t[0], 0, t[2]] for i, t in enumerate(tables)]
    rk, rv = ko.gather_tokens(bits, good, [20, 33, 40])
    sentinel = to_bits(torch.full((1,), 7.0, dtype=cache.dtype))[0]
    gk, gv = to_bits(ok)[0], to_bits(ov)[0]
    want_rows = list(range(0, 20)) + list(range(20, 36)) + list(range(52, 53)) + \
        list(range(53, 80))                             # seq 2 rows 53..92 clipped at 80
    src_rows = list(range(0, 20)) + list(range(20, 36)) + list(range(52, 53)) + \
        list(range(53, 80))
    for out, ref in ((gk, rk[0]), (gv, rv[0])):
        assert np.array_equal(out[want_rows], ref[src_rows])
        assert (out[36:52] == sentinel).all()           # the bad block's 16 tokens


def test_gather_explicit_cu_seqlens(device):
    """A caller's cu_seqlens places each sequence's rows (here with gaps and
    out of order); rows no sequence covers keep their contents."""
    rng = np.random.default_rng(34)
    N, L, H, D = 48, 2, 2, 64
    bits = random_bits(rng, (N, L, 2, 16, H, D), "bf16")
    cache = to_device_bits(bits, "bf16", device)
    lens = np.asarray([20, 5, 33], dtype=np.int64)
    tables = _tables_for(rng, lens, N)
    bt = torch.from_numpy(ko.pad_block_tables(tables)).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    starts = [70, 3, 30]                              # gaps 0..2, 8..29, 63..69
    cu = torch.tensor(starts + [120], dtype=torch.int32, device=device)
    out_k, out_v = A.gather_tokens(cache, bt, sl, 120, int(lens.max()), cu_seqlens=cu)
    rk, rv = ko.gather_tokens(bits, tables, lens)     # packed in sequence order
    packed = np.concatenate([[0], np.cumsum(lens)])
    gk, gv = to_bits(out_k), to_bits(out_v)
    for b, s in enumerate(starts):
        n = int(lens[b])
        assert np.array_equal(gk[:, s:s + n], rk[:, packed[b]:packed[b] + n]), b
        assert np.array_equal(gv[:, s:s + n], rv[:, packed[b]:packed[b] + n]), b


def test_gather_rejects_bad_metadata(device):
    """cu_seqlens of another dtype, length or device, and tables or lengths on
    the host, raise before any launch."""
    rng = np.random.default_rng(35)
    N, L, H, D = 16, 1, 2, 64
    cache = to_device_bits(random_bits(rng, (N, L, 2, 16, H, D), "bf16"), "bf16", device)
    lens = np.asarray([20, 5], dtype=np.int64)
    bt = torch.from_numpy(ko.pad_block_tables(_tables_for(rng, lens, N))).to(device)
    sl = torch.from_numpy(lens.astype(np.int32)).to(device)
    good = torch.tensor([0, 20, 25], dtype=torch.int32, device=device)
    for cu in (good.to(torch.int64), good[:2], good.cpu(), torch.cumsum(sl, 0)):
        with pytest.raises(ValueError):
            A.gather_tokens(cache, bt, sl, 25, 20, cu_seqlens=cu)
    with pytest.raises(ValueError):
        A.gather_tokens(cache, bt.cpu(), sl, 25, 20)
    with pytest.raises(ValueError):
        A.gather_tokens(cache, bt, sl.cpu(), 25, 20)
    k, v = A.gather_tokens(cache, bt, sl, 25, 20, cu_seqlens=good)
    torch.cuda.synchronize()
    assert k.shape == (1, 25, H, D)
