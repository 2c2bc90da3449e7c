"""Device-side block-id checks (iekv_check_ids) against NumPy's set arithmetic (GPU).

The kernels mark destination ids in a bitmap with atomics and probe source ids
against it; the expected verdict here comes from sorting and set membership on
the host (np.unique, np.isin), a different route to the same three facts: every
id inside its pool, no destination twice, and within one pool no block both read
and written. Lists range from empty to 300,000 ids, with problems planted at
random positions, at the first and last entry, and at the pool's edges.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from iekv import _native

pytestmark = pytest.mark.gpu


def expected_bits(src, dst, src_blocks, dst_blocks, same_pool):
    bits = 0
    if src is not None and src.size and (src.min() < 0 or src.max() >= src_blocks):
        bits |= _native.IEKV_IDS_SRC_RANGE
    if dst is not None and dst.size:
        inside = dst[(dst >= 0) & (dst < dst_blocks)]
        if inside.size != dst.size:
            bits |= _native.IEKV_IDS_DST_RANGE
        if np.unique(inside).size != inside.size:
            bits |= _native.IEKV_IDS_DST_REPEATED
        if same_pool and src is not None:
            ok_src = src[(src >= 0) & (src < src_blocks)]
            if np.isin(ok_src, inside).any():
                bits |= _native.IEKV_IDS_OVERLAP
    return bits


def pools(gpu, src_blocks, dst_blocks):
    from iekv.engine.pools import KVPool, allocate_pool

    a = KVPool(*allocate_pool(src_blocks, 4, 1, 1, 8, dtype=torch.float16, device=gpu), 4)
    b = KVPool(*allocate_pool(dst_blocks, 4, 1, 1, 8, dtype=torch.float16, device=gpu), 4)
    return a, b


def run_check(src_pool, src, dst_pool, dst):
    """Status bits of one iekv_check_ids call on the current stream."""
    n = len(dst) if dst is not None else len(src)
    s = torch.from_numpy(src.astype(np.int32)).to(src_pool.device) if src is not None else None
    d = torch.from_numpy(dst.astype(np.int32)).to(dst_pool.device) if dst is not None else None
    owner = dst_pool if dst_pool is not None else src_pool
    workspace, status = owner.check_buffers()
    status.fill_(-1)                      # the call must overwrite it
    _native.call("iekv_check_ids",
                 src_pool.native.handle if src is not None else None,
                 s.data_ptr() if s is not None else None,
                 dst_pool.native.handle if dst is not None else None,
                 d.data_ptr() if d is not None else None, n,
                 workspace.data_ptr() if dst is not None else None,
                 workspace.numel() * 4 if dst is not None else 0, status.data_ptr(),
                 torch.cuda.current_stream(owner.device).cuda_stream)
    return int(status.item())


def test_valid_lists_pass_and_every_planted_problem_is_reported(gpu):
    rng = np.random.default_rng(11)
    src_pool, dst_pool = pools(gpu, 5000, 7001)          # 7,001 bits: a partial last word
    sizes = [0, 1, 2, 31, 32, 33, 255, 256, 257, 4096, 5000]
    cases = 0
    for n in sizes:
        for plant in ("none", "src_low", "src_high", "dst_low", "dst_high", "repeat", "all"):
            src = rng.choice(5000, size=n, replace=True).astype(np.int64)
            dst = rng.permutation(7001)[:n].astype(np.int64)
            if n and plant in ("src_low", "all"):
                src[rng.integers(n)] = -1
            if n and plant in ("src_high", "all"):
                src[-1] = 5000
            if n and plant in ("dst_low", "all"):
                dst[0] = -7
            if n and plant in ("dst_high", "all"):
                dst[rng.integers(n)] = 7001
            if n > 1 and plant in ("repeat", "all"):
                i, j = rng.choice(n, size=2, replace=False)
                dst[j] = dst[i] if 0 <= dst[i] < 7001 else 6999
                dst[i] = dst[j]
            want = expected_bits(src, dst, 5000, 7001, same_pool=False)
            got = run_check(src_pool, src, dst_pool, dst)
            assert got == want, (n, plant, got, want)
            if plant == "none" or n == 0:
                assert got == 0
            cases += 1
    assert cases == len(sizes) * 7


def test_lists_of_one_kind_and_long_lists(gpu):
    rng = np.random.default_rng(12)
    src_pool, dst_pool = pools(gpu, 300_000, 300_000)
    dst = rng.permutation(300_000).astype(np.int64)
    assert run_check(None, None, dst_pool, dst) == 0               # every block once
    dst[123_456] = dst[7]
    assert run_check(None, None, dst_pool, dst) == _native.IEKV_IDS_DST_REPEATED
    src = rng.integers(0, 300_000, size=250_000)
    assert run_check(src_pool, src, None, None) == 0               # sources may repeat
    src[-1] = 300_000
    assert run_check(src_pool, src, None, None) == _native.IEKV_IDS_SRC_RANGE
    # The status is overwritten, not accumulated: a good list after a bad one reads 0.
    assert run_check(src_pool, src[:-1], None, None) == 0


def test_copies_within_one_pool_must_not_overlap(gpu):
    rng = np.random.default_rng(13)
    pool, _ = pools(gpu, 2048, 8)
    for n in (1, 64, 1000):
        ids = rng.permutation(2048)
        src, dst = ids[:n].astype(np.int64), ids[n:2 * n].astype(np.int64)
        assert run_check(pool, src, pool, dst) == 0
        src[rng.integers(n)] = dst[rng.integers(n)]
        got = run_check(pool, src, pool, dst)
        assert got == _native.IEKV_IDS_OVERLAP == expected_bits(src, dst, 2048, 2048, True)
        # The same lists between two pools are no overlap.
        other, _ = pools(gpu, 2048, 8)
        assert run_check(other, src, pool, dst) == 0


def test_the_copier_raises_for_bad_device_ids_and_moves_nothing(gpu):
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import allocate_pool

    def copier(blocks, check=True):
        k, v = allocate_pool(blocks, 4, 2, 2, 8, dtype=torch.float16, device=gpu, zero=False)
        for t in k + v:
            t.copy_(torch.randn(t.shape, device=gpu, dtype=torch.float16))
        return HipSlotCopier(k, v, 4, check_device_ids=check)

    src, dst = copier(64), copier(32)
    before = [t.clone() for t in dst.k_caches + dst.v_caches]
    ids = lambda xs: torch.tensor(xs, dtype=torch.int32, device=gpu)
    with pytest.raises(IndexError, match="source block id out of range"):
        dst.copy_blocks(src, ids([0, 64]), ids([1, 2]))
    with pytest.raises(IndexError, match="destination block id out of range"):
        dst.copy_blocks(src, ids([0, 1]), ids([1, 32]))
    with pytest.raises(ValueError, match="distinct"):
        dst.copy_blocks(src, ids([0, 1]), ids([5, 5]))
    with pytest.raises(ValueError, match="disjoint"):
        dst.copy_blocks(dst, ids([3, 4]), ids([4, 9]))
    with pytest.raises(ValueError, match="distinct"):
        dst.write_blocks(ids([2, 2]), src.read_blocks(ids([0, 1])))
    with pytest.raises(IndexError, match="source block id out of range"):
        src.read_blocks(ids([63, 64]))
    torch.cuda.synchronize()
    for a, b in zip(before, dst.k_caches + dst.v_caches):
        assert torch.equal(a, b)
    assert dst.blocks_written == 0
    # Valid device ids move as they do unchecked.
    dst.copy_blocks(src, ids([10, 11, 12]), ids([0, 31, 7]))
    torch.cuda.synchronize()
    for a, b in zip(src.k_caches + src.v_caches, dst.k_caches + dst.v_caches):
        for s_id, d_id in ((10, 0), (11, 31), (12, 7)):
            assert torch.equal(a[s_id * 4:(s_id + 1) * 4], b[d_id * 4:(d_id + 1) * 4])
    assert dst.blocks_written == 3
    # Unchecked copiers take device ids as they are (the kernels skip ids outside the pool).
    loose = copier(32, check=False)
    loose.copy_blocks(src, ids([0, 1]), ids([1, 32]))
    assert loose.blocks_written == 2


def test_two_copiers_over_one_cache_are_one_pool(gpu):
    """The engine makes several copiers over the same caches (transfer, offload,
    swap). A direct copy between two of them is a copy within one pool: sources that
    overlap destinations are refused for host lists, long host tables and checked
    device ids alike, and nothing moves. Caches that overlap without being the same
    arrays are refused as well."""
    from iekv.engine.copier import HipSlotCopier
    from iekv.engine.pools import allocate_pool

    k, v = allocate_pool(600, 4, 2, 2, 8, dtype=torch.float16, device=gpu, zero=False)
    for t in k + v:
        t.copy_(torch.randn(t.shape, device=gpu, dtype=torch.float16))
    a = HipSlotCopier(k, v, 4, check_device_ids=True)
    b = HipSlotCopier(k, v, 4, check_device_ids=True)
    assert a.pool.native.handle.value != b.pool.native.handle.value
    assert a.pool.memory_relation(b.pool) == "same"
    before = [t.clone() for t in k + v]
    with pytest.raises(ValueError, match="disjoint|both"):
        b.copy_blocks(a, [3, 4], [4, 9])                        # host list: the library
    with pytest.raises(ValueError, match="disjoint"):
        b.copy_blocks(a, list(range(0, 600)), list(range(599, -1, -1)))   # long: NumPy
    ids = lambda xs: torch.tensor(xs, dtype=torch.int32, device=gpu)
    with pytest.raises(ValueError, match="disjoint"):
        b.copy_blocks(a, ids([3, 4]), ids([4, 9]))               # device ids, checked on GPU
    torch.cuda.synchronize()
    for x, y in zip(before, k + v):
        assert torch.equal(x, y)
    # disjoint blocks move between the two handles as within one
    b.copy_blocks(a, [1, 2], [7, 8])
    torch.cuda.synchronize()
    for t in k + v:
        assert torch.equal(t[7 * 4:9 * 4], t[1 * 4:3 * 4])
    # a view of the caches shifted by one block overlaps them without being them
    shifted = HipSlotCopier([t[4:] for t in k], [t[4:] for t in v], 4)
    assert shifted.pool.memory_relation(a.pool) == "partial"
    with pytest.raises(ValueError, match="overlap in memory"):
        shifted.copy_blocks(a, [1], [2])


def test_the_checks_at_the_top_of_a_pool_of_int32_max_blocks(gpu):
    """A pool of INT32_MAX blocks (16-byte tiles, one layer: 64 GiB; a 256 MiB
    bitmap): ids next to the int32 limit land in the bitmap's last word, and each
    check still tells them apart: a valid same-pool list passes, a destination
    repeated at the top, a source that is also a destination at the top, and ids
    just outside the pool at either end are each reported."""
    from iekv.engine.pools import KVPool, allocate_pool

    n = 2**31 - 1
    top = n - 1
    pool = KVPool(*allocate_pool(n, 1, 1, 1, 16, dtype=torch.uint8, device=gpu, zero=False), 1)
    a = np.array
    cases = [   # (sources, destinations, expected bits), one pool
        (a([top, top - 2, 3]), a([top - 1, 0, top - 3]), 0),
        (a([top, top - 2]), a([top - 1, top - 1]), _native.IEKV_IDS_DST_REPEATED),
        (a([top, 5]), a([top - 1, top]), _native.IEKV_IDS_OVERLAP),
        (a([top, 5]), a([n, 7]), _native.IEKV_IDS_DST_RANGE),
        (a([-1, 5]), a([top, 7]), _native.IEKV_IDS_SRC_RANGE),
    ]
    for src, dst, bits in cases:
        print(f"int32-limit id check {src.tolist()} -> {dst.tolist()}", flush=True)
        assert expected_bits(src, dst, n, n, True) == bits
        assert run_check(pool, src, pool, dst) == bits, (src, dst)
    pool.native.close()
    del pool
    torch.cuda.empty_cache()
