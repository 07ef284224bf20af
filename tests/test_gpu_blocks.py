"""GPU parity of block movement: swap (aegaeon.ops.swap, aegaeon/ops/swap.cu:25-59),
pack/scatter, pool copy and defrag — bit-exact against the oracle and the
golden fixture."""
import numpy as np
import pytest
import torch

from aegaeon_amd import ops
from oracle import kv_oracle as ko
from tests.kvtest_utils import load_golden, random_bits, to_bits, to_device_bits

pytestmark = pytest.mark.gpu


def _tiny_cache(device):
    z = load_golden()
    N, L, H, D, BS = (int(x) for x in z["geometry"])
    pool = z["pool"].copy()
    pool[z["append_idx"]] = z["append_val"]
    cache = to_device_bits(pool, "fp16", device).view(N, L, 2, BS, H, D)
    return z, cache


@pytest.mark.parametrize("staging", ["auto", None, "small"])
def test_swap_out_golden(device, staging):
    z, cache = _tiny_cache(device)
    n = len(z["swap_src"])
    host = torch.zeros((n, *cache.shape[1:]), dtype=cache.dtype, pin_memory=True)
    stg = torch.empty(3 * ops.block_bytes_of(cache), dtype=torch.uint8, device=device) \
        if staging == "small" else staging
    ops.swap(z["swap_src"].tolist(), z["swap_dst"].tolist(), False, cache, host, staging=stg)
    torch.cuda.synchronize()
    got = host.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    assert np.array_equal(got, z["host_after_swap"])


@pytest.mark.parametrize("staging", ["auto", None, "small"])
def test_swap_round_trip(device, staging):
    """swap-out then swap-in into a different set of free blocks reproduces the
    original bytes under the re-indexing (closed form)."""
    rng = np.random.default_rng(7)
    N, shape = 96, (3, 2, 16, 2, 64)
    bits = random_bits(rng, (N, *shape), "bf16")
    cache = to_device_bits(bits, "bf16", device)
    used = rng.permutation(N)[:40]
    free = np.setdiff1d(np.arange(N), used)
    rng.shuffle(free)
    back = free[:40]
    cpu_ids = np.concatenate([np.arange(10, 30), np.arange(50, 70)])  # two host runs
    host = torch.zeros((80, *shape), dtype=torch.bfloat16, pin_memory=True)
    stg = torch.empty(3 * ops.block_bytes_of(cache), dtype=torch.uint8, device=device) \
        if staging == "small" else staging
    ops.swap(used, cpu_ids, False, cache, host, staging=stg)
    ops.swap(cpu_ids, back, True, cache, host, staging=stg)
    torch.cuda.synchronize()
    got = to_bits(cache)
    ref = bits.copy()
    host_ref = np.zeros((80, *shape), dtype=np.uint16)
    ko.swap_blocks(used, cpu_ids, False, ref, host_ref)
    ko.swap_blocks(cpu_ids, back, True, ref, host_ref)
    assert np.array_equal(got, ref)
    assert np.array_equal(host.view(torch.int16).numpy().view(np.uint16), host_ref)
    assert np.array_equal(got[back], bits[used])


@pytest.mark.parametrize("block_bytes", [16, 8192, 16384, 16400, 917504])
def test_pack_scatter_copy(device, block_bytes):
    rng = np.random.default_rng(block_bytes)
    N = 48 if block_bytes < 500000 else 24
    pool_np = rng.integers(0, 256, size=(N, block_bytes), dtype=np.uint8)
    pool = torch.from_numpy(pool_np).to(device)
    ids = rng.permutation(N)[: N // 2]
    staged = ops.pack_blocks(pool, ids)
    assert np.array_equal(staged.cpu().numpy(), ko.pack_blocks(pool_np, ids))
    dst_ids = rng.permutation(N)[: N // 2]
    other = torch.zeros_like(pool)
    ops.scatter_blocks(staged, dst_ids, other)
    ref = np.zeros_like(pool_np)
    ko.scatter_blocks(ko.pack_blocks(pool_np, ids), dst_ids, ref)
    assert np.array_equal(other.cpu().numpy(), ref)
    # pool-to-pool copy with both id lists
    third = torch.zeros_like(pool)
    ops.copy_blocks(pool, third, ids, dst_ids)
    ref3 = np.zeros_like(pool_np)
    ko.copy_blocks(pool_np, ref3, ids, dst_ids)
    assert np.array_equal(third.cpu().numpy(), ref3)


@pytest.mark.parametrize("block_bytes", [16400, 917504])
def test_copy_without_id_lists(device, block_bytes):
    """aegkv_copy_blocks with both id lists null copies blocks 0..n-1 of one pool
    into another (the C ABI's identity form; partial last tile at 16400 bytes),
    leaving the blocks past n untouched."""
    from aegaeon_amd import _lib
    rng = np.random.default_rng(block_bytes + 1)
    N, n = 12, 7
    src_np = rng.integers(0, 256, size=(N, block_bytes), dtype=np.uint8)
    src = torch.from_numpy(src_np).to(device)
    dst = torch.full_like(src, 0xA5)
    rc = _lib.load().aegkv_copy_blocks(src.data_ptr(), N, dst.data_ptr(), N, None, None, n,
                                       block_bytes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    ref = np.full_like(src_np, 0xA5)
    ref[:n] = src_np[:n]
    assert np.array_equal(dst.cpu().numpy(), ref)


def test_defrag_in_place(device):
    rng = np.random.default_rng(3)
    N, bb = 200, 4096
    pool_np = rng.integers(0, 256, size=(N, bb), dtype=np.uint8)
    live = rng.permutation(N)[:90]
    tables = [list(map(int, live[i:i + 10])) for i in range(0, 90, 10)]
    src, dst = ko.plan_defrag(live, list(range(N)))
    pool = torch.from_numpy(pool_np).to(device)
    ops.defrag_blocks(pool, src, dst)
    got = pool.cpu().numpy()
    new_tables = ko.apply_defrag(tables, src, dst)
    assert sorted(x for t in new_tables for x in t) == list(range(90))
    for old, new in zip(tables, new_tables):
        assert np.array_equal(got[new], pool_np[old])


def test_empty_lists_are_noops(device):
    cache = torch.zeros((4, 2, 16, 1, 64), dtype=torch.float16, device=device)
    host = torch.zeros((4, 2, 16, 1, 64), dtype=torch.float16, pin_memory=True)
    ops.swap([], [], False, cache, host)
    ops.defrag_blocks(cache, [], [])
    torch.cuda.synchronize()


from hypothesis import given, settings, HealthCheck, strategies as st  # noqa: E402


@st.composite
def _swap_case(draw):
    n_pool = draw(st.integers(4, 48))
    n = draw(st.integers(1, n_pool // 2))
    layers = draw(st.integers(1, 3))
    heads = draw(st.sampled_from([1, 2, 4]))
    dim = draw(st.sampled_from([8, 64, 128]))
    perm = draw(st.permutations(range(n_pool)))
    n_host = draw(st.integers(n, 2 * n + 8))
    host_ids = draw(st.permutations(range(n_host)))[:n]
    if draw(st.booleans()):  # runs of consecutive host ids (one DMA each)
        start = draw(st.integers(0, n_host - n))
        host_ids = list(range(start, start + n))
    staging = draw(st.sampled_from(["auto", None, 1, 3]))
    seed = draw(st.integers(0, 2 ** 31 - 1))
    return n_pool, (layers, 2, 16, heads, dim), perm[:n], perm[n:2 * n], host_ids, n_host, \
        staging, seed


@settings(max_examples=25, deadline=None, suppress_health_check=[HealthCheck.too_slow,
                                                                  HealthCheck.function_scoped_fixture])
@given(case=_swap_case())
def test_swap_round_trip_property(device, case):
    """Random pools, id permutations, host id runs and staging sizes: the
    swap-out leaves host[host_ids[i]] == cache[src[i]] bit for bit, the swap-in
    to fresh ids brings every block back, and untouched blocks keep their bytes."""
    n_pool, shape, src, back, host_ids, n_host, staging, seed = case
    rng = np.random.default_rng(seed)
    bits = random_bits(rng, (n_pool, *shape), "fp16")
    cache = to_device_bits(bits, "fp16", device)
    host = torch.zeros((n_host, *shape), dtype=torch.float16, pin_memory=True)
    stg = staging
    if isinstance(staging, int):
        stg = torch.empty(staging * ops.block_bytes_of(cache), dtype=torch.uint8, device=device)
    ops.swap(src, host_ids, False, cache, host, staging=stg)
    torch.cuda.synchronize()
    hb = host.view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(hb[host_ids], bits[src])
    others = np.setdiff1d(np.arange(n_host), host_ids)
    assert not hb[others].any()
    ops.swap(host_ids, back, True, cache, host, staging=stg)
    torch.cuda.synchronize()
    got = to_bits(cache)
    ref, host_ref = bits.copy(), np.zeros((n_host, *shape), dtype=np.uint16)
    ko.swap_blocks(src, host_ids, False, ref, host_ref)
    ko.swap_blocks(host_ids, back, True, ref, host_ref)
    assert np.array_equal(got, ref)
    assert np.array_equal(got[back], bits[src])
    untouched = np.setdiff1d(np.arange(n_pool), back)
    assert np.array_equal(got[untouched], bits[untouched])
