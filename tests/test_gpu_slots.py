"""Slot scatter (write_kv) and paged gather (gather_context) kernels vs the NumPy oracle (GPU)."""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.slots import gather_context, write_kv

pytestmark = pytest.mark.gpu

CASES = [  # block_size, heads, dim, dtype
    (16, 8, 128, torch.bfloat16),
    (16, 2, 16, torch.float32),
    (4, 1, 2, torch.float32),
    (3, 1, 5, torch.float16),     # 10-byte rows: 2-byte vectors
    (16, 8, 128, torch.float8_e4m3fn),
    (5, 3, 3, torch.uint8),       # 9-byte rows
    (4, 16, 128, torch.float32),  # 8 KiB rows: two steps of four vectors per lane
    (2, 9, 128, torch.float32),   # 4.5 KiB rows: a full step, then 32 lanes
]


def as_np(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.uint8).cpu().numpy().copy()


def random_pool(num_blocks, bs, heads, dim, dtype, device, layers=2, seed=0):
    from iekv.engine.pools import KVPool, allocate_pool

    k, v = allocate_pool(num_blocks, bs, layers, heads, dim, dtype=dtype, device=device,
                         zero=False)
    k[0]._base.view(torch.uint8).random_(0, 256,
                                          generator=torch.Generator(device).manual_seed(seed))
    return k, v, KVPool(k, v, bs)


def random_rows(n, heads, dim, dtype, device, seed):
    raw = torch.randint(0, 256, (n, heads, dim * torch.tensor([], dtype=dtype).element_size()),
                        dtype=torch.uint8, device=device,
                        generator=torch.Generator(device).manual_seed(seed))
    return raw.view(dtype)


@pytest.mark.parametrize("bs,heads,dim,dtype", CASES)
def test_write_slots_matches_write_kv(gpu, bs, heads, dim, dtype):
    from iekv.engine.slots import write_slots

    k, v, pool = random_pool(20, bs, heads, dim, dtype, gpu, seed=1)
    oracle_k = [as_np(t) for t in k]
    oracle_v = [as_np(t) for t in v]
    rng = np.random.default_rng(2)
    slots = [int(s) for s in rng.permutation(20 * bs)[:13]]
    for layer in range(2):
        kr = random_rows(13, heads, dim, dtype, gpu, seed=10 + layer)
        vr = random_rows(13, heads, dim, dtype, gpu, seed=20 + layer)
        write_slots(pool, layer, kr, vr, slots)
        write_kv(as_np(kr), as_np(vr), oracle_k[layer], oracle_v[layer], slots)
    torch.cuda.synchronize()
    for got, want in zip(k + v, oracle_k + oracle_v):
        assert np.array_equal(as_np(got), want)


@pytest.mark.parametrize("bs,heads,dim,dtype", CASES)
def test_gather_rows_matches_gather_context(gpu, bs, heads, dim, dtype):
    from iekv.engine.slots import gather_rows

    k, v, pool = random_pool(20, bs, heads, dim, dtype, gpu, seed=3)
    rng = np.random.default_rng(4)
    for context_len in (1, bs, 3 * bs + 1, 7 * bs):
        needed = -(-context_len // bs)
        table = [int(b) for b in rng.permutation(20)[:needed]] + [-1, -1]  # padded like layouts
        for array, cache in enumerate(k + v):
            got = gather_rows(pool, array, table, context_len)
            want = gather_context(as_np(cache), table, context_len, bs)
            assert np.array_equal(as_np(got), want), (context_len, array)


@pytest.mark.parametrize("bs,heads,dim,dtype", CASES)
def test_one_launch_writes_every_layer_like_write_kv_per_layer(gpu, bs, heads, dim, dtype):
    """iekv_write_slots_layers: all four layers at once, then layers 1..2 with new
    rows, then (layer_stride 0) the same rows into every layer; each against the
    oracle's write_kv per layer."""
    from iekv import _native
    from iekv.engine.slots import write_slots_layers

    L = 4
    k, v, pool = random_pool(20, bs, heads, dim, dtype, gpu, layers=L, seed=5)
    oracle_k = [as_np(t) for t in k]
    oracle_v = [as_np(t) for t in v]
    rng = np.random.default_rng(6)
    for first, n_layers, seed in ((0, L, 30), (1, 2, 40)):
        slots = [int(x) for x in rng.permutation(20 * bs)[:13]]
        kr = random_rows(n_layers * 13, heads, dim, dtype, gpu, seed).view(n_layers, 13, heads, dim)
        vr = random_rows(n_layers * 13, heads, dim, dtype, gpu, seed + 1).view(
            n_layers, 13, heads, dim)
        write_slots_layers(pool, kr, vr, slots, first_layer=first)
        for l in range(n_layers):
            write_kv(as_np(kr[l]), as_np(vr[l]), oracle_k[first + l], oracle_v[first + l], slots)
    slots = [int(x) for x in rng.permutation(20 * bs)[:7]]
    kr, vr = (random_rows(7, heads, dim, dtype, gpu, seed) for seed in (50, 51))
    dev_slots = torch.tensor(slots, dtype=torch.int64, device=gpu)
    _native.call("iekv_write_slots_layers", pool.native.handle, 0, L, bs, kr.data_ptr(),
                 vr.data_ptr(), 0, dev_slots.data_ptr(), 7,
                 torch.cuda.current_stream().cuda_stream)
    for l in range(L):
        write_kv(as_np(kr), as_np(vr), oracle_k[l], oracle_v[l], slots)
    torch.cuda.synchronize()
    for got, want in zip(k + v, oracle_k + oracle_v):
        assert np.array_equal(as_np(got), want)


@pytest.mark.parametrize("bs,heads,dim,dtype", CASES)
def test_one_launch_gathers_every_array_like_gather_context(gpu, bs, heads, dim, dtype):
    from iekv.engine.slots import gather_rows_arrays

    k, v, pool = random_pool(20, bs, heads, dim, dtype, gpu, layers=3, seed=7)
    rng = np.random.default_rng(8)
    for context_len in (1, bs, 3 * bs + 1, 7 * bs):
        needed = -(-context_len // bs)
        table = [int(b) for b in rng.permutation(20)[:needed]] + [-1]
        got = gather_rows_arrays(pool, table, context_len)
        assert got.shape[:2] == (6, context_len)
        for array, cache in enumerate(k + v):
            want = gather_context(as_np(cache), table, context_len, bs)
            assert np.array_equal(as_np(got[array]), want), (context_len, array)
        part = gather_rows_arrays(pool, table, context_len, first_array=2, n_arrays=3)
        assert torch.equal(part.view(torch.uint8), got[2:5].contiguous().view(torch.uint8))


def test_slot_calls_validate_before_launch(gpu):
    from iekv.engine.slots import gather_rows, write_slots

    k, v, pool = random_pool(4, 4, 1, 2, torch.float32, gpu)
    rows = torch.zeros(2, 1, 2, device=gpu)
    with pytest.raises(IndexError):
        write_slots(pool, 0, rows, rows, [0, 16])
    with pytest.raises(IndexError):
        write_slots(pool, 2, rows, rows, [0, 1])
    with pytest.raises(ValueError):
        write_slots(pool, 0, rows, rows, [0])
    with pytest.raises(IndexError):
        gather_rows(pool, 0, [3], 6)
    from iekv.engine.slots import gather_rows_arrays, write_slots_layers

    with pytest.raises(IndexError):
        write_slots_layers(pool, rows[None].expand(2, -1, -1, -1), rows[None].expand(2, -1, -1, -1),
                           [0, 1], first_layer=1)
    with pytest.raises(IndexError):
        gather_rows_arrays(pool, [0, 1], 6, first_array=3, n_arrays=2)


@pytest.mark.parametrize("cache_dtype", [torch.float32, torch.bfloat16], ids=str)
def test_the_model_decodes_identically_through_the_slot_kernels(gpu, cache_dtype):
    from conftest import golden
    from iekv.engine.engine import Engine, EngineConfig
    from iekv.engine.toy_model import ModelConfig, ToyTransformer
    from iekv.serve.disaggregated import DisaggregatedEngine

    g = golden("disaggregation")
    cfg = EngineConfig(**g["engine"])

    def model(hip_kv):
        return ToyTransformer(ModelConfig(**g["model"]), seed=g["model_seed"], device=gpu,
                              cache_dtype=cache_dtype, hip_kv=hip_kv)

    torch_path = Engine(model(False), cfg).generate(g["prompts"], max_new_tokens=6,
                                                    temperature=0.0)
    hip_colocated = Engine(model(True), cfg).generate(g["prompts"], max_new_tokens=6,
                                                      temperature=0.0)
    hip_split = DisaggregatedEngine(model(True), cfg, mode="direct").generate(
        g["prompts"], max_new_tokens=6, temperature=0.0)
    assert hip_colocated == torch_path == hip_split


def test_slots_and_table_entries_at_the_top_of_a_pool_of_int32_max_blocks(gpu):
    """A pool of INT32_MAX blocks of 2 slots (8-byte rows, one layer's K and V: 64 GiB)
    has 2^32 - 2 slots: write_kv's int64 slots above 2^32 - 5 and past 2^31, and
    gather_context's table entries next to INT32_MAX, address rows 32 GiB into each
    array. Both kernels move exactly those rows, and the rows beside each written one
    keep their bytes."""
    from iekv.engine.pools import KVPool, allocate_pool
    from iekv.engine.slots import gather_rows_arrays, write_slots_layers

    n, bs = 2**31 - 1, 2
    rows = n * bs
    k, v = allocate_pool(n, bs, 1, 1, 8, dtype=torch.uint8, device=gpu, zero=False)
    pool = KVPool(k, v, bs)
    gen = torch.Generator(gpu).manual_seed(71)
    slots = [rows - 1, rows - 4, 5, 2**31 + 7, 2**32 - 9]
    beside = sorted({s + d for s in slots for d in (-1, 1) if 0 <= s + d < rows} - set(slots))
    idx = torch.tensor(beside, dtype=torch.long, device=gpu)
    for arr in (k[0], v[0]):
        arr.view(rows, 8).index_copy_(0, idx, torch.randint(
            0, 256, (len(beside), 8), dtype=torch.uint8, device=gpu, generator=gen))
    kept = [arr.view(rows, 8)[idx].clone() for arr in (k[0], v[0])]
    new_k = torch.randint(0, 256, (1, len(slots), 1, 8), dtype=torch.uint8, device=gpu,
                          generator=gen)
    new_v = torch.randint(0, 256, (1, len(slots), 1, 8), dtype=torch.uint8, device=gpu,
                          generator=gen)
    print("int32-limit slot pool: write_kv", flush=True)
    write_slots_layers(pool, new_k, new_v, slots)
    torch.cuda.synchronize()
    sl = torch.tensor(slots, dtype=torch.long, device=gpu)
    assert torch.equal(k[0].view(rows, 8)[sl], new_k[0].view(-1, 8))
    assert torch.equal(v[0].view(rows, 8)[sl], new_v[0].view(-1, 8))
    for arr, before in zip((k[0], v[0]), kept):
        assert torch.equal(arr.view(rows, 8)[idx], before)
    # gather_context over a table whose blocks sit at the top of the pool
    table = [n - 1, n - 2, 3, n - 5]
    context = 7                                          # the last block half used
    want_rows = torch.tensor([table[j // bs] * bs + j % bs for j in range(context)],
                             dtype=torch.long, device=gpu)
    for arr in (k[0], v[0]):
        arr.view(rows, 8).index_copy_(0, want_rows, torch.randint(
            0, 256, (context, 8), dtype=torch.uint8, device=gpu, generator=gen))
    print("int32-limit slot pool: gather_context", flush=True)
    out = gather_rows_arrays(pool, table, context)
    torch.cuda.synchronize()
    for a, arr in enumerate((k[0], v[0])):
        assert torch.equal(out[a].view(context, 8), arr.view(rows, 8)[want_rows])
    pool.native.close()
    del k, v, pool, out
    torch.cuda.empty_cache()


def test_gather_takes_the_block_table_as_a_list_or_a_tensor(gpu):
    """A decode loop may keep its block tables on the GPU or in a CPU tensor:
    gather_context and the every-array gather read the same rows through a device
    int32 or int64 tensor, a CPU tensor and a Python list, and a table too short
    for the context raises IndexError in every form, as the reference's does."""
    from iekv.engine.slots import gather_rows, gather_rows_arrays

    bs, heads, dim = 4, 2, 16
    k, v, pool = random_pool(30, bs, heads, dim, torch.float16, gpu, seed=91)
    table, context = [17, 2, 29, 8], 14
    raw = lambda t: t.view(torch.uint8)       # NaN bit patterns compare as bytes
    want = gather_rows_arrays(pool, table, context)
    for form in (torch.tensor(table, dtype=torch.int32, device=gpu),
                 torch.tensor(table, dtype=torch.int64, device=gpu),
                 torch.tensor(table, dtype=torch.int32)):
        assert torch.equal(raw(gather_rows_arrays(pool, form, context)), raw(want))
        for array in (0, 3):
            assert torch.equal(raw(gather_rows(pool, array, form, context)), raw(want[array]))
        with pytest.raises(IndexError):
            gather_rows_arrays(pool, form[:3], context)
        with pytest.raises(IndexError):
            gather_rows(pool, 0, form[:3], context)
    oracle = gather_context(as_np(k[1]), table, context, bs)
    assert np.array_equal(as_np(want[1]), oracle.reshape(as_np(want[1]).shape))
