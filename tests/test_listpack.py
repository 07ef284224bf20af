"""The request-list packer behind prepare_model_inputs (CPU): the same arrays
as numpy builds from the lists, and the errors the reference's own list walk
(worker.py:596-646) would hit as Python exceptions."""
import numpy as np
import pytest

from aegaeon_amd import _listpack


def test_tables_pack_like_numpy():
    rng = np.random.default_rng(7)
    tables = [rng.integers(0, 2 ** 31 - 1, int(n)).tolist() for n in rng.integers(0, 40, 200)]
    tables[3] = []
    ids, off = _listpack.pack_tables(tables)
    ids = np.frombuffer(ids, dtype=np.int32)
    off = np.frombuffer(off, dtype=np.int64)
    assert off[0] == 0 and np.array_equal(np.diff(off), [len(t) for t in tables])
    assert np.array_equal(ids, np.concatenate([np.asarray(t, dtype=np.int64) for t in tables]))
    # tuples, and an empty batch
    ids2, off2 = _listpack.pack_tables(tuple(tuple(t) for t in tables))
    assert ids2 == ids.tobytes() and off2 == off.tobytes()
    ids3, off3 = _listpack.pack_tables([])
    assert len(ids3) == 0 and np.frombuffer(off3, dtype=np.int64).tolist() == [0]


def test_requests_pack_like_numpy():
    reqs = [(0, [5, 6, 7], 3, 0), (1, [9], 11, 10), (2, [], 4, 4), (3, (1, 2), 2, 0)]
    seq, ctx, tok = _listpack.pack_requests(reqs)
    assert np.frombuffer(seq, dtype=np.int32).tolist() == [3, 11, 4, 2]
    assert np.frombuffer(ctx, dtype=np.int32).tolist() == [0, 10, 4, 0]
    assert np.frombuffer(tok, dtype=np.int64).tolist() == [5, 6, 7, 9, 1, 2]
    big = [(0, [2 ** 40], 1, 0)]
    assert np.frombuffer(_listpack.pack_requests(big)[2], dtype=np.int64).tolist() == [2 ** 40]


def test_errors():
    with pytest.raises(ValueError):  # two tokens for one new position
        _listpack.pack_requests([(0, [1, 2], 5, 4)])
    with pytest.raises(TypeError):
        _listpack.pack_requests([(0, [1])])
    with pytest.raises(TypeError):
        _listpack.pack_tables([[1, "2"]])
    with pytest.raises(TypeError):
        _listpack.pack_tables([3])
    with pytest.raises(OverflowError):
        _listpack.pack_tables([[2 ** 31]])
    with pytest.raises(OverflowError):
        _listpack.pack_requests([(0, [], 2 ** 31, 2 ** 31)])
