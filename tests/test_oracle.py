"""Pin the NumPy oracle before it is trusted as the checker of the HIP path.

Checks, each chosen so a plausible mistake in the oracle fails one of them:
* the reference's layout known-answer tests (tests/test_paged_attention.py:54-70)
  re-run through the oracle's block addressing;
* the closed form of a handoff (target tiles equal, everything else untouched);
* the golden digests the reference itself produced for the cfg1 handoff;
* planted mistakes (off-by-one span, K/V swap, layer reversal, stale read)
  that those checks must catch.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest

from conftest import golden
from helpers import cfg1_inputs
from oracle.copier import LayeredSlotCopier, handoff, pack, packed_image, unpack


def slot_numbered_cache(num_blocks, block_size, heads=1, dim=2, dtype=np.float32):
    cache = np.zeros((num_blocks * block_size, heads, dim), dtype=dtype)
    for slot in range(cache.shape[0]):
        cache[slot, 0, 0] = slot
    return cache


def test_read_block_addresses_the_gather_context_known_answer():
    # Reference KAT: table [3, 1], bs 4, context 6 -> slots [12,13,14,15,4,5].
    cache = slot_numbered_cache(8, 4)
    copier = LayeredSlotCopier([cache], [cache.copy()], 4)
    k3, _ = copier.read_block(3)
    k1, _ = copier.read_block(1)
    gathered = np.concatenate([k3[0], k1[0]])[:6, 0, 0]
    assert list(gathered) == [12, 13, 14, 15, 4, 5]


def test_write_block_lands_on_the_slots_of_its_block():
    # Slots are rows (reference KAT: write_kv to slots [9, 0, 5] writes rows 9, 0, 5).
    k = np.zeros((16, 1, 2), dtype=np.float32)
    v = np.zeros_like(k)
    copier = LayeredSlotCopier([k], [v], 4)
    tile = np.arange(8, dtype=np.float32).reshape(4, 1, 2) + 1
    copier.write_block(2, ([tile], [-tile]))
    assert np.array_equal(k[8:12], tile) and np.array_equal(v[8:12], -tile)
    assert not k[:8].any() and not k[12:].any()


def test_read_returns_a_snapshot_not_a_view():
    k = slot_numbered_cache(4, 4)
    copier = LayeredSlotCopier([k], [k.copy()], 4)
    payload = copier.read_block(1)
    k[4:8] = -1
    assert list(payload[0][0][:, 0, 0]) == [4, 5, 6, 7]


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.uint16, np.uint8, np.int8])
def test_handoff_closed_form(dtype):
    rng = np.random.default_rng(7)
    layers, bs, heads, dim, n_src, n_dst = 3, 4, 2, 8, 40, 50
    shape = (n_src * bs, heads, dim)

    def fill(shape):
        if np.dtype(dtype).kind == "f":
            return rng.standard_normal(shape).astype(dtype)
        info = np.iinfo(dtype)
        return rng.integers(info.min, info.max, size=shape, endpoint=True).astype(dtype)

    src_k = [fill(shape) for _ in range(layers)]
    src_v = [fill(shape) for _ in range(layers)]
    dst_k = [fill((n_dst * bs, heads, dim)) for _ in range(layers)]
    dst_v = [fill((n_dst * bs, heads, dim)) for _ in range(layers)]
    before_src = [a.copy() for a in src_k + src_v]
    before_dst = [a.copy() for a in dst_k + dst_v]
    src_tables = [list(rng.permutation(n_src)[:7]), list(rng.permutation(n_src)[:5])]
    chosen = rng.permutation(n_dst)[:12]
    dst_tables = [list(chosen[:7]), list(chosen[7:])]
    handoff(LayeredSlotCopier(src_k, src_v, bs), LayeredSlotCopier(dst_k, dst_v, bs),
            src_tables, dst_tables)
    for a, (src, dst) in enumerate(zip(src_k + src_v, dst_k + dst_v)):
        assert np.array_equal(src.view(np.uint8), before_src[a].view(np.uint8))
        touched = set()
        for s_tab, d_tab in zip(src_tables, dst_tables):
            for s, d in zip(s_tab, d_tab):
                touched.add(int(d))
                assert dst[d * bs:(d + 1) * bs].tobytes() == src[s * bs:(s + 1) * bs].tobytes()
        for d in set(range(n_dst)) - touched:
            assert dst[d * bs:(d + 1) * bs].tobytes() == before_dst[a][d * bs:(d + 1) * bs].tobytes()


def test_packed_image_orders_k_layers_then_v_layers():
    layers, bs = 3, 2
    k = [np.full((4 * bs, 1, 1), 10 + l, dtype=np.uint8) for l in range(layers)]
    v = [np.full((4 * bs, 1, 1), 20 + l, dtype=np.uint8) for l in range(layers)]
    image = packed_image(pack(LayeredSlotCopier(k, v, bs), [1, 3]))
    assert image.shape == (2, 2 * layers, bs)
    assert list(image[0, :, 0]) == [10, 11, 12, 20, 21, 22]


def cfg1_oracle_run(copier_cls=LayeredSlotCopier):
    g = golden("cfg1_handoff")
    lengths, src_tables, k, v = cfg1_inputs()
    dst_k = [np.zeros_like(a) for a in k]
    dst_v = [np.zeros_like(a) for a in v]
    src = copier_cls(k, v, 16)
    dst = copier_cls(dst_k, dst_v, 16)
    digest = hashlib.sha256()
    for s_tab, d_tab in zip(src_tables, g["dst_tables"]):
        payloads = pack(src, s_tab)
        digest.update(packed_image(payloads).tobytes())
        unpack(dst, d_tab, payloads)
    return g, lengths, src_tables, (k, v), (dst_k, dst_v), src, dst, digest.hexdigest()


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def test_cfg1_oracle_reproduces_the_reference_digests():
    g, lengths, src_tables, (k, v), (dk, dv), src, dst, packed = cfg1_oracle_run()
    assert lengths == g["lengths"] and src_tables == g["src_tables"]
    assert [sha(a) for a in k] == g["src_sha256"]["k"]
    assert [sha(a) for a in v] == g["src_sha256"]["v"]
    assert [sha(a) for a in dk] == g["dst_sha256"]["k"]
    assert [sha(a) for a in dv] == g["dst_sha256"]["v"]
    assert packed == g["packed_sha256"]
    assert src.blocks_read == g["src_counters"]["blocks_read"] == g["total_blocks"]
    assert src.bytes_moved == g["src_counters"]["bytes_moved"]
    assert dst.blocks_written == g["dst_counters"]["blocks_written"]
    assert dst.bytes_moved == g["dst_counters"]["bytes_moved"]


class OffByOneSpan(LayeredSlotCopier):
    def _span(self, block_id):
        first = block_id * self.block_size + 1
        return slice(first, first + self.block_size)


class SwappedKV(LayeredSlotCopier):
    def write_block(self, block_id, payload):
        k, v = payload
        super().write_block(block_id, (v, k))


class ReversedLayers(LayeredSlotCopier):
    def read_block(self, block_id):
        k, v = super().read_block(block_id)
        return k[::-1], v[::-1]


class StaleRead(LayeredSlotCopier):
    """Returns views instead of snapshots."""

    def read_block(self, block_id):
        rows = self._span(block_id)
        self.blocks_read += 1
        return [c[rows] for c in self.k_caches], [c[rows] for c in self.v_caches]


@pytest.mark.parametrize("planted", [OffByOneSpan, SwappedKV, ReversedLayers])
def test_planted_mistakes_fail_the_golden_digests(planted):
    try:
        g, *_, (dk, dv), _src, _dst, packed = cfg1_oracle_run(planted)
    except ValueError:
        return  # the mistake broke the run outright (a short slice at the pool's end)
    ok = ([sha(a) for a in dk] == g["dst_sha256"]["k"]
          and [sha(a) for a in dv] == g["dst_sha256"]["v"] and packed == g["packed_sha256"])
    assert not ok


def test_a_planted_stale_read_fails_the_snapshot_check():
    k = slot_numbered_cache(4, 4)
    payload = StaleRead([k], [k.copy()], 4).read_block(1)
    k[4:8] = -1
    assert list(payload[0][0][:, 0, 0]) != [4, 5, 6, 7]


def test_slot_oracle_reproduces_the_reference_known_answers():
    from oracle.slots import gather_context, write_kv

    cache = slot_numbered_cache(8, 4)
    gathered = gather_context(cache, [3, 1], 6, 4)
    assert list(gathered[:, 0, 0]) == [12, 13, 14, 15, 4, 5]
    k_cache = np.zeros((16, 1, 2), dtype=np.float32)
    v_cache = np.zeros_like(k_cache)
    k = np.arange(6, dtype=np.float32).reshape(3, 1, 2)
    write_kv(k, k, k_cache, v_cache, [9, 0, 5])
    assert np.array_equal(k_cache[9], k[0]) and np.array_equal(k_cache[0], k[1])
    assert np.array_equal(k_cache[5], k[2])
    with pytest.raises(ValueError):
        write_kv(k, k, k_cache, v_cache, [0, 1])
    with pytest.raises(IndexError):
        gather_context(cache, [3], 6, 4)
