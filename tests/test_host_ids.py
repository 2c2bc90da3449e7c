"""Host block ids: the library's checks of host-id calls against the pool's NumPy checks.

A serving loop hands the copier short Python tables; those go to the library's
host-id entry points unconverted by NumPy (``_host_id_array``), and the library
checks them (IEKV_ERR_RANGE for an id outside the pool, IEKV_ERR_IDS for a
destination given twice or a copy within one pool whose sources overlap its
destinations), which Python raises as IndexError / ValueError like the NumPy
checks of ``KVPool.host_ids``. For every table, both must accept or refuse alike.

No kernel runs: the pools are registered on a device that does not exist (their
arrays are equally spaced, so registering touches no GPU), so a call whose ids
pass every check stops at the device switch with IEKV_ERR_HIP.
"""
import ctypes
from types import SimpleNamespace

import numpy as np
import pytest

from iekv import _native
from iekv.engine.copier import HOST_IDS_MAX, _host_id_array, issue_order
from iekv.engine.pools import KVPool

NO_DEVICE = 99


def pool(num_blocks, tile=64, arrays=2, base=1 << 30):
    ptrs = [base + a * num_blocks * tile for a in range(arrays)]
    return _native.Pool(ptrs, tile_bytes=tile, num_blocks=num_blocks, device=NO_DEVICE)


def library_outcome(fn, *args):
    """"pass" when every id check passed (the call then fails at the device switch),
    else the exception type the id check raised."""
    try:
        _native.call(fn, *args)
    except (_native.NativeIndexError, _native.NativeValueError) as e:
        assert isinstance(e, (IndexError, ValueError)) and isinstance(e, RuntimeError)
        return "IndexError" if isinstance(e, IndexError) else "ValueError"
    except _native.NativeError as e:
        assert e.code == _native.IEKV_ERR_HIP, str(e)
        return "pass"
    raise AssertionError("a call on a device that does not exist succeeded")


def numpy_outcome(check):
    try:
        check()
    except IndexError:
        return "IndexError"
    except ValueError:
        return "ValueError"
    return "pass"


def addr(a):
    return a.buffer_info()[0]


def test_short_lists_become_int32_arrays_and_the_rest_stays_with_numpy():
    assert list(_host_id_array([3, 1, 2])) == [3, 1, 2]
    assert list(_host_id_array((np.int64(7), True, -1))) == [7, 1, -1]   # the library checks
    assert len(_host_id_array([])) == 0
    assert len(_host_id_array(list(range(HOST_IDS_MAX)))) == HOST_IDS_MAX
    assert _host_id_array(list(range(HOST_IDS_MAX + 1))) is None     # uploaded instead
    assert _host_id_array(np.arange(3)) is None
    assert _host_id_array([1.0, 2.0]) is None                            # not integers
    assert _host_id_array([1 << 40]) is None                             # not 32-bit


@pytest.mark.parametrize("seed", range(4))
def test_direct_copy_ids_are_refused_alike_by_the_library_and_numpy(seed):
    rng = np.random.default_rng(seed)
    for case in range(300):
        num_blocks = int(rng.integers(2, 40))
        n = int(rng.integers(0, 10)) if case % 5 else int(rng.integers(200, 700))
        src = [int(x) for x in rng.integers(-1, num_blocks + 1, size=n)]
        if rng.integers(2):     # distinct, sometimes one past either end of the pool
            dst = [int(x) for x in rng.permutation(max(n, num_blocks + 1))[:n]
                   - rng.integers(0, 2)]
        else:                   # repeats likely
            dst = [int(x) for x in rng.integers(0, num_blocks, size=n)]
        assert len(src) == len(dst) == n
        same = bool(rng.integers(3) == 0)
        a = pool(num_blocks)
        # one pool: the same handle, or a second handle over the same arrays
        b = (a if rng.integers(2) else pool(num_blocks)) if same else \
            pool(num_blocks, base=1 << 31)
        s, d = _host_id_array(src), _host_id_array(dst)
        if s is None or d is None:
            continue
        got = library_outcome("iekv_copy_direct_ids", a.handle, b.handle, addr(s), addr(d),
                              n, None)

        def numpy_check():
            ss, dd = issue_order(src, dst)
            ss = KVPool.host_ids(SimpleNamespace(num_blocks=num_blocks), ss, what="source block")
            dd = KVPool.host_ids(SimpleNamespace(num_blocks=num_blocks), dd, unique=True,
                                 what="destination block", ascending=True)
            if same and np.isin(ss, dd).any():
                raise ValueError("overlap")

        assert got == numpy_outcome(numpy_check), (src, dst, same, num_blocks)
        a.close()
        if b is not a:
            b.close()


@pytest.mark.parametrize("seed", range(3))
def test_pack_and_unpack_ids_are_refused_alike_by_the_library_and_numpy(seed):
    rng = np.random.default_rng(100 + seed)
    for _ in range(200):
        num_blocks = int(rng.integers(2, 30))
        n = int(rng.integers(1, 12))
        ids = [int(x) for x in rng.integers(-1, num_blocks + 1, size=n)]
        p = pool(num_blocks)
        h = _host_id_array(ids)
        staging = np.zeros(n * p.block_bytes, dtype=np.uint8)
        sp = staging.__array_interface__["data"][0]
        fake = SimpleNamespace(num_blocks=num_blocks)
        got = library_outcome("iekv_pack_ids", p.handle, addr(h), n, sp, staging.size, None)
        assert got == numpy_outcome(lambda: KVPool.host_ids(fake, ids)), ids
        got = library_outcome("iekv_unpack_ids", p.handle, addr(h), n, sp, staging.size, None)
        assert got == numpy_outcome(lambda: KVPool.host_ids(fake, ids, unique=True)), ids
        p.close()


@pytest.mark.parametrize("seed", range(3))
def test_host_tier_ids_are_refused_alike_by_the_library_and_numpy(seed):
    """iekv_offload_ids and iekv_offload_blocks_ids check their source ids for
    range; iekv_restore_ids and
    iekv_restore_blocks_ids check their destination ids for range and repeats,
    as the pool's NumPy checks do."""
    rng = np.random.default_rng(200 + seed)
    for _ in range(150):
        num_blocks = int(rng.integers(2, 30))
        n = int(rng.integers(1, 12))
        ids = [int(x) for x in rng.integers(-1, num_blocks + 1, size=n)]
        p = pool(num_blocks)
        h = _host_id_array(ids)
        image = np.zeros(n * p.block_bytes, dtype=np.uint8)
        ip = image.__array_interface__["data"][0]
        staging = np.zeros(p.block_bytes, dtype=np.uint8)
        sp = staging.__array_interface__["data"][0]
        images = (ctypes.c_void_p * n)(*[ip + i * p.block_bytes for i in range(n)])
        fake = SimpleNamespace(num_blocks=num_blocks)
        got = library_outcome("iekv_offload_ids", p.handle, addr(h), n, ip, image.size, sp,
                              staging.size, None, None)
        assert got == numpy_outcome(lambda: KVPool.host_ids(fake, ids)), ids
        want = numpy_outcome(lambda: KVPool.host_ids(fake, ids, unique=True))
        got = library_outcome("iekv_restore_ids", p.handle, addr(h), n, ip, image.size, sp,
                              staging.size, None, None)
        assert got == want, ids
        got = library_outcome("iekv_restore_blocks_ids", p.handle, addr(h), n, images, sp,
                              staging.size, None, None)
        assert got == want, ids
        got = library_outcome("iekv_offload_blocks_ids", p.handle, addr(h), n, images, sp,
                              staging.size, None, None)
        assert got == numpy_outcome(lambda: KVPool.host_ids(fake, ids)), ids
        p.close()


def test_the_library_names_the_offending_id():
    p, q = pool(16), pool(16)
    tables = {name: _host_id_array(t) for name, t in
              {"a": [0, 1], "b": [3, 16], "c": [0, 1, 2], "d": [5, 9, 5], "e": [4, 1],
               "f": [2, 4]}.items()}       # held here: the library reads them during the call
    with pytest.raises(IndexError, match=r"destination block id 16 \(entry 1\) out of range"):
        _native.call("iekv_copy_direct_ids", p.handle, q.handle, addr(tables["a"]),
                     addr(tables["b"]), 2, None)
    with pytest.raises(ValueError, match=r"destination block ids must be distinct \(id 5 given"):
        _native.call("iekv_copy_direct_ids", p.handle, q.handle, addr(tables["c"]),
                     addr(tables["d"]), 3, None)
    with pytest.raises(ValueError, match=r"disjoint source and destination blocks \(block 4 is"):
        _native.call("iekv_copy_direct_ids", p.handle, p.handle, addr(tables["e"]),
                     addr(tables["f"]), 2, None)
    p.close()
    q.close()


def test_non_integer_ids_are_refused_not_truncated():
    """The reference slices with ``b * bs`` (ie/engine/copier.py:14-16), which refuses a
    float id; NumPy's int64 conversion would truncate it to a real block instead."""
    import torch

    from iekv.engine.pools import integer_ids

    for bad in ([1.5], np.array([2.0]), torch.tensor([3.0]), [1, 2.5], np.array(["4"]),
                [None]):
        with pytest.raises(TypeError):
            integer_ids(bad)
        with pytest.raises(TypeError):
            issue_order(bad, [0] * len(bad))
    assert list(integer_ids([3, np.int32(1), True])) == [3, 1, 1]      # ints and bools
    assert list(integer_ids(np.array([7], dtype=np.uint16))) == [7]
    assert list(integer_ids(torch.tensor([5, 6], dtype=torch.int32))) == [5, 6]
    assert integer_ids([]).size == 0 and integer_ids(np.array([])).size == 0
