"""Seeded synthetic workloads: geometry, distributions and the seed-0 sizes the
byte counts of the benchmark are quoted on."""
import numpy as np

from aegaeon_amd import workloads as W


def test_block_bytes_of_the_model_shapes():
    # (L, 2, 16, Hkv, D) x 2 bytes (aegaeon/aegaeon/config.py:256-271)
    assert W.TINY.block_bytes == 8192
    assert W.QWEN25_7B.block_bytes == 917504
    assert W.YI15_9B.block_bytes == 1572864
    assert W.LLAMA2_13B.block_bytes == 13107200
    assert W.QWEN25_7B.bytes_per_token == 57344  # 2*28*4*128*2, the GQA-true value


def test_tiny_case_fits_its_pool():
    wb = W.tiny_batch(0)
    assert wb.batch == 8 and wb.n_pool_blocks == 64
    assert ((wb.context_lens >= 1) & (wb.context_lens <= 128)).all()
    assert wb.n_blocks_used <= 64
    ids = [b for t in wb.block_tables for b in t]
    assert len(set(ids)) == len(ids)
    # each table covers context_len + 1 tokens
    for t, c in zip(wb.block_tables, wb.context_lens):
        assert len(t) == -(-(int(c) + 1) // 16)


def test_qwen_append_batch_seed0():
    wb = W.qwen_append_batch(0)
    assert wb.batch == 256
    assert abs(wb.context_lens.mean() - 585.7) < 0.1
    assert wb.n_blocks_used == 9507 and wb.n_pool_blocks == 19014
    assert wb.append_bytes() == 2 * 256 * 28 * 2 * 4 * 128 * 2 + 8 * 256 == 29362176
    s = wb.slot_mapping()
    assert len(np.unique(s)) == 256 and (s >= 0).all() and (s < 19014 * 16).all()


def test_qwen_attention_batch_seed0():
    wb = W.qwen_attention_batch(0)
    assert wb.batch == 128
    assert int(wb.seq_lens.sum()) == 189059
    assert wb.seq_lens.min() >= 16 and wb.seq_lens.max() <= 8192
    assert wb.attention_bytes() == 389075836


def test_lognormal_mean_is_the_arithmetic_mean():
    rng = np.random.default_rng(0)
    x = W.lognormal_lengths(rng, 200000, 600.0, 1.0, 1, 10 ** 9)
    assert abs(x.mean() / 600.0 - 1) < 0.02


def test_llama_swap_workload():
    wl = W.llama_swap_workload(0)
    assert wl.n_blocks == 4096 and wl.n_pool_blocks == 8192
    assert not set(wl.gpu_ids) & set(wl.swap_in_ids)
    assert len(set(wl.swap_in_ids)) == 4096
    assert wl.pack_bytes() == 2 * 4096 * 13107200 + 8 * 4096


def test_unified_pool_slabs_hold_one_shape_each():
    wl = W.unified_pool_workload(0)
    for name, g in wl.geometries.items():
        valid = set(wl.valid_ids(name))
        live = [b for t in wl.tables[name] for b in t]
        assert set(live) <= valid and len(set(live)) == len(live)
        assert len(live) <= len(valid) // 2 + 1
        # byte ranges of live blocks stay inside their own slabs
        for b in live[:50]:
            s = b * g.block_bytes // wl.slab_bytes
            assert wl.slab_owner[s] == name
            assert (b + 1) * g.block_bytes <= (s + 1) * wl.slab_bytes


def test_plan_compaction_matches_oracle_and_invariants():
    from aegaeon_amd.pool import plan_compaction, remap_tables, slab_of, slab_range
    from oracle import kv_oracle as ko
    import pytest
    rng = np.random.default_rng(0)
    for trial in range(20):
        valid = np.sort(rng.permutation(1000)[:300])
        live = rng.permutation(valid)[:rng.integers(0, 301)]
        src, dst = plan_compaction(live, valid)
        osrc, odst = ko.plan_defrag(live, valid.tolist())
        assert src.tolist() == list(osrc) and dst.tolist() == list(odst)
        t = remap_tables([live.tolist()], src, dst)[0]
        assert sorted(t) == valid[:len(live)].tolist()
    with pytest.raises(ValueError):
        plan_compaction([5, 5], list(range(10)))
    with pytest.raises(ValueError):
        plan_compaction([11], list(range(10)))
    # slab geometry of the reference's 1 GiB slabs (block_manager.py:242-245)
    S, bb = 1 << 30, 917504
    a, b = slab_range(1, S, bb)
    assert a * bb >= S and b * bb <= 2 * S and (b + 1) * bb > 2 * S
    assert all(slab_of(x, S, bb) == 1 for x in (a, b - 1))
