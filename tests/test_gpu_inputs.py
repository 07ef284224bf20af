"""GPU parity of the device-side input preparation against the oracle's
restatement of Worker._prepare_model_inputs (aegaeon/aegaeon/worker.py:596-676).
Every output is integer: the bar is bit-exact equality of values and dtypes."""
import numpy as np
import pytest
import torch

from aegaeon_amd import inputs as I
from aegaeon_amd._lib import AegkvError
from aegaeon_amd.workloads import qwen_append_batch
from oracle import kv_oracle as ko

pytestmark = pytest.mark.gpu


def _compare(dev_out, ref):
    toks, pos, md = dev_out
    torch.cuda.synchronize()
    assert np.array_equal(toks.cpu().numpy(), ref["input_tokens"])
    assert np.array_equal(pos.cpu().numpy(), ref["input_positions"])
    for k in ("slot_mapping", "seq_lens_tensor", "context_lens_tensor", "query_start_loc",
              "seq_start_loc", "block_tables"):
        got = md[k].cpu().numpy()
        assert got.dtype == ref[k].dtype, k
        assert np.array_equal(got, ref[k]), k
    for k in ("num_prefills", "num_prefill_tokens", "num_decode_tokens", "seq_lens",
              "max_query_len", "max_prefill_seq_len", "max_decode_seq_len"):
        assert md[k] == ref[k], k


def _mixed_batch(rng, n_prefill, n_decode, pool=65536):
    """Prefills (context 0, several tokens) then decodes (one token), tables
    drawn from a permutation of the pool, as the block manager hands out."""
    perm = iter(rng.permutation(pool).tolist())
    reqs, tables = [], []
    for i in range(n_prefill):
        n = int(rng.integers(1, 300))
        reqs.append((i, rng.integers(0, 32000, n).tolist(), n, 0))
        tables.append([next(perm) for _ in range(-(-n // 16))])
    for i in range(n_decode):
        ctx = int(rng.integers(1, 2000))
        reqs.append((n_prefill + i, [int(rng.integers(0, 32000))], ctx + 1, ctx))
        # tables may hold more blocks than the sequence needs (pre-allocated)
        tables.append([next(perm) for _ in range(-(-(ctx + 1) // 16) + int(rng.integers(0, 2)))])
    return reqs, tables


@pytest.mark.parametrize("n_prefill,n_decode", [(0, 1), (1, 0), (3, 5), (0, 64), (8, 200)])
def test_matches_oracle(device, n_prefill, n_decode):
    rng = np.random.default_rng(n_prefill * 1000 + n_decode)
    reqs, tables = _mixed_batch(rng, n_prefill, n_decode)
    _compare(I.prepare_model_inputs(reqs, tables, device), ko.prepare_model_inputs(reqs, tables))


def test_lengths_at_block_edges(device):
    """Positions 15/16/17 and 31/32 straddle block boundaries."""
    reqs = [(0, [1], 16, 15), (1, [2], 17, 16), (2, [3], 18, 17), (3, [4], 33, 32),
            (4, [5, 6], 17, 15)]
    tables = [[7], [8, 9], [10, 11], [12, 13, 14], [15, 16]]
    _compare(I.prepare_model_inputs(reqs, tables, device), ko.prepare_model_inputs(reqs, tables))


def test_qwen_decode_batch(device):
    """The Qwen2.5-7B decode step: 256 requests, lognormal context lengths."""
    wb = qwen_append_batch(0)
    reqs = I.decode_requests(wb.context_lens)
    _compare(I.prepare_model_inputs(reqs, wb.block_tables, device),
             ko.prepare_model_inputs(reqs, wb.block_tables))
    # the slot mapping equals the workload's own (worker.py:628-633)
    _, _, md = I.prepare_model_inputs(reqs, wb.block_tables, device)
    assert np.array_equal(md["slot_mapping"].cpu().numpy(), wb.slot_mapping())


def test_short_table_raises(device):
    with pytest.raises(AegkvError):
        I.prepare_model_inputs([(0, [1], 17, 16)], [[3]], device)


def test_arrays_from_block_manager(device):
    """Block tables straight from the native block manager's flat layout give
    the same outputs as the list path and the oracle."""
    from aegaeon_amd.block_manager import BlockManager
    rng = np.random.default_rng(17)
    bm = BlockManager(0, 1)
    bm.register_gpu_space(0, 4096, (28, 2, 16, 4, 128))
    ctx = rng.integers(1, 900, 40)
    rids = list(range(40))
    bm.allocate_blocks_by_count(rids, [int(-(-(c + 1) // 16)) for c in ctx], 0)
    for r in rids[::3]:                                  # scatter the free list
        bm.free_blocks(r)
    bm.allocate_blocks_by_count(rids[::3], [int(-(-(ctx[r] + 1) // 16)) for r in rids[::3]], 0)
    offsets, ids = bm.flat_block_tables(rids)
    reqs = I.decode_requests(ctx)
    tokens = np.asarray([r[1][0] for r in reqs], dtype=np.int64)
    got = I.prepare_inputs_from_arrays(ids, offsets, ctx + 1, ctx, tokens, device)
    tables = [bm.get_block_table(r).blocks for r in rids]
    _compare(got, ko.prepare_model_inputs(reqs, tables))
