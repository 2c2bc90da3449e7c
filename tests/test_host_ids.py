"""Host-side id checks: the plain-Python path for short tables against the NumPy path.

``KVPool.short_host_ids`` and ``short_issue_order`` take a serving loop's short
block tables without NumPy; for every input they accept they must give what
``KVPool.host_ids`` and ``issue_order`` give, and raise what those raise. Both
are pure host logic, so they run here on pools described by a block count.
"""
from types import SimpleNamespace

import numpy as np
import pytest

from iekv import _native
from iekv.engine.copier import issue_order, short_issue_order
from iekv.engine.pools import KVPool


def pool(num_blocks):
    return SimpleNamespace(num_blocks=num_blocks)


def outcome(fn, *args, **kwargs):
    try:
        return "ok", np.asarray(fn(*args, **kwargs), dtype=np.int64).reshape(-1).tolist()
    except (IndexError, ValueError) as e:
        return type(e).__name__, str(e)


@pytest.mark.parametrize("seed", range(6))
def test_short_tables_are_checked_like_the_numpy_path(seed):
    rng = np.random.default_rng(seed)
    for _ in range(400):
        num_blocks = int(rng.integers(1, 40))
        n = int(rng.integers(0, 12))
        ids = [int(x) for x in rng.integers(-2, num_blocks + 2, size=n)]
        kind = rng.integers(2)
        table = ids if kind else tuple(ids)
        unique = bool(rng.integers(2))
        p = pool(num_blocks)
        short = outcome(KVPool.short_host_ids, p, table, unique=unique, what="x")
        ref = outcome(KVPool.host_ids, p, table, unique=unique, what="x")
        assert short == ref, (table, unique, num_blocks)


def test_short_tables_take_only_short_lists_of_integers():
    p = pool(1000)
    assert KVPool.short_host_ids(p, np.arange(3)) is None            # arrays: NumPy path
    assert KVPool.short_host_ids(p, [1.0, 2.0]) is None              # floats: NumPy path
    assert KVPool.short_host_ids(p, list(range(_native.INLINE_IDS + 1))) is None
    got = KVPool.short_host_ids(p, list(range(_native.INLINE_IDS)))
    assert list(got) == list(range(_native.INLINE_IDS))
    assert list(KVPool.short_host_ids(p, [np.int64(7), True])) == [7, 1]
    assert len(KVPool.short_host_ids(p, [])) == 0
    with pytest.raises(IndexError, match="id 1000 out of range"):
        KVPool.short_host_ids(p, [3, 1000])
    with pytest.raises(IndexError, match="id -1 out of range"):
        KVPool.short_host_ids(p, (-1, 5))
    with pytest.raises(ValueError, match="must be distinct"):
        KVPool.short_host_ids(p, [4, 4], unique=True)
    assert list(KVPool.short_host_ids(p, [4, 4])) == [4, 4]          # repeats allowed for sources


@pytest.mark.parametrize("seed", range(4))
def test_short_issue_order_sorts_like_issue_order(seed):
    rng = np.random.default_rng(seed)
    for _ in range(300):
        n = int(rng.integers(0, 20))
        dst = [int(x) for x in rng.permutation(64)[:n]]
        src = [int(x) for x in rng.integers(0, 64, size=n)]
        s, d = short_issue_order(src, dst)
        rs, rd = issue_order(src, dst)
        assert s == rs.tolist() and d == rd.tolist()
    with pytest.raises(ValueError, match="3 source blocks for 2 destinations"):
        short_issue_order([1, 2, 3], [4, 5])
    with pytest.raises(ValueError, match="3 source blocks for 2 destinations"):
        issue_order([1, 2, 3], [4, 5])
    assert short_issue_order(np.arange(2), [1, 2]) is None
    assert short_issue_order([1] * 300, [2] * 300) is None
