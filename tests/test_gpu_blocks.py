"""GPU parity of block movement: swap (aegaeon.ops.swap, aegaeon/ops/swap.cu:25-59),
pack/scatter, pool copy and defrag — bit-exact against the oracle and the
golden fixture."""
import numpy as np
import pytest
import torch

from aegaeon_amd import ops
from aegaeon_amd.workloads import pinnable_blocks
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


def test_more_blocks_than_one_launch(device):
    """70,000 blocks of 16 and of 1040 bytes (a full and a partial 1 KiB tile):
    the copy kernel's grid holds at most 65,535 blocks, so the host issues
    several launches with offset id lists and offset identity sides; pack,
    scatter and the two-list copy against the oracle."""
    for bb in (16, 1040):
        rng = np.random.default_rng(bb + 70000)
        N, n = 150000, 70000
        pool_np = rng.integers(0, 256, size=(N, bb), dtype=np.uint8)
        pool = torch.from_numpy(pool_np).to(device)
        ids = rng.permutation(N)[:n]
        staged = ops.pack_blocks(pool, ids)
        want = ko.pack_blocks(pool_np, ids)
        assert np.array_equal(staged.cpu().numpy(), want)
        dst_ids = rng.permutation(N)[:n]
        other = torch.zeros_like(pool)
        ops.scatter_blocks(staged, dst_ids, other)
        ref = np.zeros_like(pool_np)
        ko.scatter_blocks(want, dst_ids, ref)
        assert np.array_equal(other.cpu().numpy(), ref)
        third = torch.zeros_like(pool)
        ops.copy_blocks(pool, third, ids, dst_ids)
        assert np.array_equal(third.cpu().numpy(), ref)


def test_contiguous_copy_past_one_grid_row(device):
    """An identity copy of 32 GiB + 1 MiB: more 1 KiB tiles (33,555,456) than one
    grid row holds (2^31 work-items / 64 = 33,554,432), so the row's workgroups
    loop over the rest.  Checked on the GPU: every byte, by comparing the two
    buffers, after filling the source with random words."""
    free, _ = torch.cuda.mem_get_info(device)
    nbytes = (32 << 30) + (1 << 20)
    if free < 2 * nbytes + (4 << 30):
        pytest.skip("needs 68 GB of free device memory")
    src = torch.empty(nbytes // 4, dtype=torch.int32, device=device)
    src.random_()
    dst = torch.zeros_like(src)
    ops.copy_blocks(src.view(torch.uint8).view(1, nbytes), dst.view(torch.uint8).view(1, nbytes),
                    None, None)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    del src, dst
    torch.cuda.empty_cache()


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


def test_llama_full_size_swap_round_trip(device):
    """Llama-2-13B at full size (40 layers, 40 kv heads, D 128, fp16, 32
    sequences of 2048 tokens = 4096 blocks of 12.5 MiB in a pool of 8192):
    pack the scattered blocks, scatter them into a disjoint seeded free set,
    and check bit-exactness block by block on both sides; then a sampled host
    leg (64 blocks) through ops.swap out to pinned memory and back in.  The
    property (a move reproduces its bytes and touches nothing else) holds
    at any size; this runs it at the workload's."""
    from aegaeon_amd.workloads import llama_swap_workload
    wl = llama_swap_workload(0)
    bb = wl.geometry.block_bytes
    need = (wl.n_pool_blocks + wl.n_blocks) * bb
    torch.cuda.empty_cache()
    if torch.cuda.get_device_properties(device).total_memory < need + (16 << 30):
        pytest.skip("needs %d GiB of device memory" % ((need >> 30) + 16))
    pool = torch.empty((wl.n_pool_blocks, bb), dtype=torch.uint8, device=device)
    pool.view(torch.int32).random_(generator=torch.Generator(device=device).manual_seed(5))
    src = np.asarray(wl.gpu_ids, dtype=np.int64)
    dst = np.asarray(wl.swap_in_ids, dtype=np.int64)
    assert not set(src.tolist()) & set(dst.tolist())
    untouched = np.setdiff1d(np.arange(wl.n_pool_blocks), np.concatenate([src, dst]))
    keep = torch.from_numpy(untouched[:64]).to(device)
    before = pool[keep].clone()
    staging = ops.pack_blocks(pool, src)
    ops.scatter_blocks(staging, dst, pool)
    torch.cuda.synchronize()
    for c in range(0, wl.n_blocks, 256):
        i = torch.arange(c, min(c + 256, wl.n_blocks), device=device)
        assert torch.equal(pool[torch.from_numpy(dst[c:c + 256]).to(device)], staging[i])
        assert torch.equal(pool[torch.from_numpy(src[c:c + 256]).to(device)], staging[i])
    assert torch.equal(pool[keep], before)
    del staging
    # host leg on a sample: out to pinned memory, back in to other free ids
    n_s = 64
    host = torch.zeros((n_s, bb), dtype=torch.uint8, pin_memory=True)
    ops.swap(src[:n_s], np.arange(n_s), False, pool, host)
    ops.swap(np.arange(n_s), dst[n_s:2 * n_s], True, pool, host)
    torch.cuda.synchronize()
    assert torch.equal(host.to(device), pool[torch.from_numpy(src[:n_s]).to(device)])
    assert torch.equal(pool[torch.from_numpy(dst[n_s:2 * n_s]).to(device)],
                       pool[torch.from_numpy(src[:n_s]).to(device)])
    del pool, host, before
    torch.cuda.empty_cache()


def test_unified_pool_full_size_defrag(device):
    """The unified pool at full size (44 GiB: Yi-1.5-9B, Qwen2.5-7B and
    Llama-2-13B blocks in 1 GiB slabs, 50% live): each model's live blocks are
    compacted into the dense prefix of its id space.  Every live block's bytes
    reappear, bit-exact, at its remapped id, the new ids form the prefix, and
    the free blocks that received nothing keep their bytes."""
    from aegaeon_amd.pool import plan_compaction, remap_tables
    from aegaeon_amd.workloads import unified_pool_workload
    wl = unified_pool_workload(0)
    torch.cuda.empty_cache()
    if torch.cuda.get_device_properties(device).total_memory < 2 * wl.pool_bytes + (16 << 30):
        pytest.skip("needs %d GiB of device memory" % ((2 * wl.pool_bytes >> 30) + 16))
    pool = torch.empty(wl.pool_bytes, dtype=torch.uint8, device=device)
    pool.view(torch.int32).random_(generator=torch.Generator(device=device).manual_seed(6))
    before = pool.clone()

    def blocks(t, bb):
        nb = wl.pool_bytes // bb
        return t[:nb * bb].view(nb, bb)

    def same(a_ids, b_ids, bb):
        a_ids, b_ids = np.asarray(a_ids, dtype=np.int64), np.asarray(b_ids, dtype=np.int64)
        for c in range(0, len(a_ids), 128):
            ia = torch.from_numpy(a_ids[c:c + 128]).to(device)
            ib = torch.from_numpy(b_ids[c:c + 128]).to(device)
            if not torch.equal(blocks(pool, bb)[ia], blocks(before, bb)[ib]):
                return False
        return True

    moved = 0
    for name, g in wl.geometries.items():
        bb = g.block_bytes
        valid = list(wl.valid_ids(name))
        src, dst = plan_compaction([b for t in wl.tables[name] for b in t], valid)
        ops.defrag_blocks(pool, src, dst, block_bytes=bb)
        torch.cuda.synchronize()
        moved += len(src)
        tables = remap_tables(wl.tables[name], src, dst)
        old_ids = [b for t in wl.tables[name] for b in t]
        new_ids = [b for t in tables for b in t]
        assert sorted(new_ids) == valid[:len(new_ids)], name
        assert same(new_ids, old_ids, bb), name
        free = sorted(set(valid) - set(old_ids) - set(int(x) for x in dst))
        assert same(free, free, bb), name
    assert moved == 2047 + 2332 + 499
    del pool, before
    torch.cuda.empty_cache()


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


def test_swap_rejects_pageable_or_foreign_buffers(device):
    """A pageable swap space (every DMA would block) and staging on the host
    raise before anything is enqueued; the pool is untouched."""
    cache = torch.zeros((4, 2, 16, 1, 64), dtype=torch.float16, device=device)
    pageable = torch.zeros((4, 2, 16, 1, 64), dtype=torch.float16)
    with pytest.raises(ValueError):
        ops.swap([0, 1], [2, 3], False, cache, pageable)
    pinned = torch.zeros_like(pageable).pin_memory()
    with pytest.raises(ValueError):
        ops.swap([0, 1], [2, 3], False, cache, pinned, staging=torch.empty(1 << 16,
                                                                           dtype=torch.uint8))
    ops.swap([0, 1], [2, 3], False, cache, pinned)
    torch.cuda.synchronize()
    assert torch.equal(pinned[2:], cache[:2].cpu())


_LLAMA_BB = 40 * 2 * 16 * 40 * 128 * 2
_N_HOST = pinnable_blocks(_LLAMA_BB, 4096)


@pytest.mark.parametrize("n_host", [_N_HOST], ids=[f"{_N_HOST}of4096blocks"])
def test_llama_swap_through_pinned_host(device, n_host):
    """The Llama-2-13B swap as the worker runs it (worker.py:753-762): n_host
    of the workload's 4096 scattered 12.5 MiB blocks (all of them when the
    host can pin 64 GiB; the test id states the count) go out to a pinned host
    pool through ops.swap (staged pack, one DMA per host run) and come back
    through ops.swap into a disjoint seeded free set.  Checked bit for bit on
    both sides: the host pool against the source blocks (read back with a
    plain copy), the swapped-in blocks against the source blocks, and blocks
    no move touched against a snapshot."""
    if n_host == 0:
        pytest.skip("the host cannot pin even one 12.5 MiB block")
    from aegaeon_amd.workloads import llama_swap_workload
    wl = llama_swap_workload(0)
    bb = wl.geometry.block_bytes
    assert bb == _LLAMA_BB
    torch.cuda.empty_cache()
    if torch.cuda.get_device_properties(device).total_memory < wl.n_pool_blocks * bb + (16 << 30):
        pytest.skip("needs %d GiB of device memory" % ((wl.n_pool_blocks * bb >> 30) + 16))
    pool = torch.empty((wl.n_pool_blocks, bb), dtype=torch.uint8, device=device)
    pool.view(torch.int32).random_(generator=torch.Generator(device=device).manual_seed(8))
    src = np.asarray(wl.gpu_ids[:n_host], dtype=np.int64)
    dst = np.asarray(wl.swap_in_ids[:n_host], dtype=np.int64)
    host_ids = np.asarray(wl.cpu_ids[:n_host], dtype=np.int64)
    untouched = np.setdiff1d(np.arange(wl.n_pool_blocks), np.concatenate([src, dst]))
    keep = torch.from_numpy(untouched[::max(1, len(untouched) // 64)][:64]).to(device)
    before = pool[keep].clone()
    host = torch.empty((n_host, bb), dtype=torch.uint8, pin_memory=True)
    print(f"swap-out of {n_host} blocks ({n_host * bb / 2**30:.1f} GiB)", flush=True)
    ops.swap(src, host_ids, False, pool, host)
    ops.swap(host_ids, dst, True, pool, host)
    torch.cuda.synchronize()
    step = 128
    for c in range(0, n_host, step):
        s = torch.from_numpy(src[c:c + step]).to(device)
        d = torch.from_numpy(dst[c:c + step]).to(device)
        h = host[c:c + step].to(device)            # host rows c.. hold host ids c.. (a run)
        assert torch.equal(h, pool[s]), c
        assert torch.equal(pool[d], pool[s]), c
    assert torch.equal(pool[keep], before)
    del pool, host, before
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()


def test_calls_enqueued_far_ahead_of_the_device(device):
    """48 packs of 16384 ids each (six times the library's first id upload
    ring) enqueued behind a held stream: the host does not wait for the device
    (the ring grows instead of waiting for slices the device has not read),
    and every pack reads its own ids."""
    torch.cuda.synchronize()
    n_blocks, n, calls = 1 << 20, 16384, 48
    gen = torch.Generator(device=device).manual_seed(11)
    pool = torch.randint(-2**31, 2**31 - 1, (n_blocks, 4), dtype=torch.int32, device=device,
                         generator=gen)
    rng = np.random.default_rng(11)
    ids = [rng.choice(n_blocks, n, replace=False).astype(np.int64) for _ in range(calls)]
    outs = torch.zeros((calls, n, 4), dtype=torch.int32, device=device)
    # calibrate the spin, then hold the stream for about 300 ms
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    torch.cuda._sleep(1_000_000)
    e1.record()
    e1.synchronize()
    cycles_per_ms = 1_000_000 / max(e0.elapsed_time(e1), 1e-3)
    torch.cuda._sleep(int(300 * cycles_per_ms))
    held = torch.cuda.Event()
    held.record()
    for c in range(calls):
        ops.pack_blocks(pool, ids[c], out=outs[c])
    still_held = not held.query()
    torch.cuda.synchronize()
    for c in range(calls):
        assert torch.equal(outs[c], pool[torch.from_numpy(ids[c]).to(device)]), c
    assert still_held, "the host waited for the device while enqueueing"


@pytest.mark.parametrize("seed", [1, 2])
def test_id_lists_of_random_sizes_through_the_upload_ring(device, seed):
    """Packs and scatters with id lists of random sizes (1 to 60,000 ids),
    some enqueued behind a held stream and some not, so the upload ring wraps,
    grows and reuses slices the device has released: every call reads its own
    ids (checked against torch's gather and scatter of the same lists)."""
    torch.cuda.synchronize()
    rng = np.random.default_rng(seed)
    n_blocks = 1 << 18
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = torch.randint(-2**31, 2**31 - 1, (n_blocks, 4), dtype=torch.int32, device=device,
                         generator=gen)
    sizes = rng.integers(1, 60_000, size=40)
    ids = [rng.choice(n_blocks, int(k), replace=False).astype(np.int64) for k in sizes]
    outs = [torch.zeros((int(k), 4), dtype=torch.int32, device=device) for k in sizes]
    dst = torch.zeros_like(pool)
    for c in range(len(ids)):
        if c % 10 == 0:  # every tenth call starts behind a short hold
            torch.cuda._sleep(2_000_000)
        ops.pack_blocks(pool, ids[c], out=outs[c])
        ops.scatter_blocks(outs[c], ids[c], dst)
    torch.cuda.synchronize()
    for c in range(len(ids)):
        t = torch.from_numpy(ids[c]).to(device)
        assert torch.equal(outs[c], pool[t]), c
    touched = torch.from_numpy(np.unique(np.concatenate(ids))).to(device)
    assert torch.equal(dst[touched], pool[touched])
