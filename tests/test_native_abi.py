"""The C-ABI library loads and exports every entry point include/iekv.h declares.

No kernel runs here (no GPU is needed): only the argument checks that return
before any HIP call, which is where the ABI promises errors are raised.
"""
from __future__ import annotations

import ctypes
import re

import pytest

from conftest import ROOT

HEADER = ROOT / "include" / "iekv.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char\*)\s+(iekv_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def lib():
    from iekv import _native

    if not _native.library_path().exists():
        pytest.fail(f"{_native.library_path()} is not built (run __graft_entry__.build())")
    return _native.lib()


def test_every_declared_function_is_exported_and_bound(lib):
    from iekv import _native

    names = declared_functions()
    assert len(names) >= 10
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_native.SIGNATURES)


def test_abi_version(lib):
    assert lib.iekv_abi_version() == 21


def test_pool_create_rejects_bad_arguments_before_touching_the_gpu(lib):
    from iekv import _native

    out = ctypes.c_void_p()
    table = (ctypes.c_uint64 * 2)(4096, 4096 + 1024)
    cases = [
        (None, 2, 64, 16, "array_ptrs is null"),
        (table, 0, 64, 16, "n_arrays"),
        (table, 2, 0, 16, "tile_bytes"),
        (table, 2, 64, 0, "num_blocks"),
        (table, 2, 64, 1 << 40, "num_blocks"),
        (table, 2, 64, 17, "overlap"),          # 17 x 64 B > the 1024 B gap between arrays
    ]
    for ptrs, n, tile, blocks, message in cases:
        rc = lib.iekv_pool_create(ptrs, n, tile, blocks, 0, ctypes.byref(out))
        assert rc == _native.IEKV_ERR_INVALID
        assert message in lib.iekv_last_error().decode()
        assert not out.value


def test_calls_reject_null_pools_and_negative_counts(lib):
    from iekv import _native

    assert lib.iekv_copy_direct(None, None, None, None, 1, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_pack(None, None, 1, None, 0, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_unpack(None, None, 1, None, 0, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_offload(None, None, 1, None, 0, None, 0, None, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_restore(None, None, 1, None, 0, None, 0, None, None) == _native.IEKV_ERR_INVALID
    assert "null" in lib.iekv_last_error().decode()
    assert lib.iekv_restore_blocks(None, None, 1, None, None, 0, None, None) == \
        _native.IEKV_ERR_INVALID
    assert "null" in lib.iekv_last_error().decode()


def test_host_id_calls_check_count_and_range_before_any_launch(lib):
    """The *_ids entry points take any number of host ids (IEKV_INLINE_IDS per
    launch) and check each against its pool before anything is enqueued; a slab
    pool registers without touching the GPU."""
    from iekv import _native

    pool = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    n = _native.INLINE_IDS + 1
    ids = (ctypes.c_int32 * n)(*range(n))
    assert lib.iekv_copy_direct_ids(pool.handle, pool.handle, ids, ids, -1, None) == \
        _native.IEKV_ERR_INVALID
    assert "n_blocks is negative" in lib.iekv_last_error().decode()
    assert lib.iekv_copy_direct_ids(pool.handle, pool.handle, ids, ids, n, None) == \
        _native.IEKV_ERR_RANGE                        # a long list: every id checked
    assert "source block id 16 (entry 16)" in lib.iekv_last_error().decode()
    assert lib.iekv_pack_ids(pool.handle, None, 3, None, 0, None) == _native.IEKV_ERR_INVALID
    assert "null" in lib.iekv_last_error().decode()
    bad = (ctypes.c_int32 * 3)(0, 16, 2)
    staging = ctypes.create_string_buffer(3 * 2 * 64)
    rc = lib.iekv_unpack_ids(pool.handle, bad, 3, staging, len(staging), None)
    assert rc == _native.IEKV_ERR_RANGE
    assert "destination block id 16 (entry 1)" in lib.iekv_last_error().decode()
    rc = lib.iekv_copy_direct_ids(pool.handle, pool.handle, bad, ids, 3, None)
    assert rc == _native.IEKV_ERR_RANGE
    assert "source block id 16" in lib.iekv_last_error().decode()
    pool.close()


def test_request_lists_are_checked_before_any_launch(lib):
    """iekv_copy_direct_requests checks its counts, ids and streams first; a slab
    pool registers without touching the GPU."""
    from iekv import _native

    pool = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    h = pool.handle
    counts = (ctypes.c_int32 * 2)(1, 2)
    ids = (ctypes.c_int32 * 3)(0, 1, 2)
    streams = (ctypes.c_void_p * 1)(None)
    cases = [
        ((h, h, -1, counts, ids, ids, streams, 1, None), "n_requests is negative"),
        ((h, h, 2, None, ids, ids, streams, 1, None), "counts is null"),
        ((h, h, 2, counts, ids, ids, None, 1, None), "need at least one stream"),
        ((h, h, 2, counts, ids, ids, streams, 0, None), "need at least one stream"),
        ((h, h, 2, (ctypes.c_int32 * 2)(1, -2), ids, ids, streams, 1, None),
         "request 1 has a negative count"),
        ((h, h, 2, counts, None, ids, streams, 1, None), "source ids are null"),
        ((None, h, 2, counts, ids, ids, streams, 1, None), "null"),
    ]
    for args, message in cases:
        assert lib.iekv_copy_direct_requests(*args) == _native.IEKV_ERR_INVALID, message
        assert message in lib.iekv_last_error().decode(), message
    assert lib.iekv_copy_direct_requests(h, h, 0, None, None, None, None, 0, None) == 0
    pool.close()


def test_device_id_checks_validate_their_arguments_before_any_launch(lib):
    """iekv_check_ids needs a pool, ids for each pool it is given, a status word and,
    with a destination pool, a bitmap workspace of one bit per block."""
    from iekv import _native

    pool = _native.Pool([1 << 20, (1 << 20) + 64 * 100], tile_bytes=64, num_blocks=100,
                        device=99)
    h = pool.handle
    ids = ctypes.c_void_p(1 << 24)                  # never read: every case fails first
    status = ctypes.c_void_p(1 << 24)
    need = _native.check_workspace_bytes(100)
    assert need == 16                                # 100 bits in four 32-bit words
    cases = [
        ((None, None, None, None, 1, None, 0, status, None), _native.IEKV_ERR_INVALID,
         "no source or destination pool"),
        ((h, None, None, None, 1, None, 0, status, None), _native.IEKV_ERR_INVALID,
         "source ids are null"),
        ((None, None, h, None, 1, ids, need, status, None), _native.IEKV_ERR_INVALID,
         "destination ids are null"),
        ((h, ids, None, None, -1, None, 0, status, None), _native.IEKV_ERR_INVALID,
         "n_blocks is negative"),
        ((h, ids, None, None, 1, None, 0, None, None), _native.IEKV_ERR_INVALID,
         "status is null"),
        ((h, ids, None, None, 1, None, 0, ctypes.c_void_p((1 << 24) + 2), None),
         _native.IEKV_ERR_INVALID, "status is not 4-byte aligned"),
        ((None, None, h, ids, 1, None, need, status, None), _native.IEKV_ERR_INVALID,
         "workspace buffer is null"),
        ((None, None, h, ids, 1, ids, need - 4, status, None), _native.IEKV_ERR_CAPACITY,
         "workspace buffer holds 12 bytes, 16 needed"),
        ((None, None, h, ids, 1, ctypes.c_void_p((1 << 24) + 1), need, status, None),
         _native.IEKV_ERR_INVALID, "workspace is not 4-byte aligned"),
    ]
    for args, code, message in cases:
        assert lib.iekv_check_ids(*args) == code, message
        assert message in lib.iekv_last_error().decode(), message
    # Valid arguments reach the device switch (device 99 does not exist).
    assert lib.iekv_check_ids(h, ids, h, ids, 1, ids, need, status, None) == _native.IEKV_ERR_HIP
    assert lib.iekv_check_ids(h, ids, None, None, 0, None, 0, status, None) == \
        _native.IEKV_ERR_HIP
    pool.close()


def test_pools_are_compared_by_the_memory_they_describe(lib):
    """Two handles over one set of arrays are one pool: a host-id direct copy between
    them that uses a block as both source and destination is refused with
    IEKV_ERR_IDS, as it is through a single handle. Handles whose arrays overlap
    without being the same arrays are refused outright; separate pools pass the
    checks and reach the device switch (device 99 does not exist)."""
    from iekv import _native

    base, tile, blocks = 1 << 30, 64, 16
    stride = tile * blocks
    one = _native.Pool([base, base + stride], tile_bytes=tile, num_blocks=blocks, device=99)
    again = _native.Pool([base, base + stride], tile_bytes=tile, num_blocks=blocks, device=99)
    shifted = _native.Pool([base + tile, base + tile + stride], tile_bytes=tile,
                           num_blocks=blocks, device=99)
    apart = _native.Pool([base + 4 * stride, base + 5 * stride], tile_bytes=tile,
                         num_blocks=blocks, device=99)
    src = (ctypes.c_int32 * 2)(0, 1)
    dst = (ctypes.c_int32 * 2)(1, 2)
    for a, b in ((one, one), (one, again), (again, one)):
        assert lib.iekv_copy_direct_ids(a.handle, b.handle, src, dst, 2, None) == \
            _native.IEKV_ERR_IDS
        assert "block 1 is both" in lib.iekv_last_error().decode()
    for a, b in ((one, shifted), (shifted, again)):
        assert lib.iekv_copy_direct_ids(a.handle, b.handle, src, dst, 2, None) == \
            _native.IEKV_ERR_INVALID
        assert "overlap in memory" in lib.iekv_last_error().decode()
    assert lib.iekv_copy_direct_ids(one.handle, apart.handle, src, dst, 2, None) == \
        _native.IEKV_ERR_HIP
    status = ctypes.c_void_p(1 << 24)
    workspace = ctypes.c_void_p(1 << 24)
    need = _native.check_workspace_bytes(blocks)
    assert lib.iekv_check_ids(one.handle, src, shifted.handle, dst, 2, workspace, need, status,
                              None) == _native.IEKV_ERR_INVALID
    assert "overlap in memory" in lib.iekv_last_error().decode()
    for pool in (one, again, shifted, apart):
        pool.close()


def test_host_allocation_and_launch_floor_check_their_arguments(lib):
    """iekv_host_alloc needs an output and a positive size; a failed allocation
    leaves a null address and the runtime's message. iekv_noop needs 1 to the
    dispatch limit of workgroups and a non-negative launch count."""
    from iekv import _native

    out = ctypes.c_void_p(1234)
    assert lib.iekv_host_alloc(4096, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_host_alloc(0, ctypes.byref(out)) == _native.IEKV_ERR_INVALID
    assert not out.value and "bytes must be positive" in lib.iekv_last_error().decode()
    rc = lib.iekv_host_alloc(4096, ctypes.byref(out))
    if rc == _native.IEKV_OK:           # a machine with a GPU
        assert out.value
        assert lib.iekv_host_free(out) == _native.IEKV_OK
    else:
        assert rc == _native.IEKV_ERR_HIP and not out.value
        assert "hipHostMalloc of 4096 bytes" in lib.iekv_last_error().decode()
    assert lib.iekv_host_free(None) == _native.IEKV_OK
    assert lib.iekv_noop(0, 1, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_noop(1 << 24, 1, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_noop(1, -1, None) == _native.IEKV_ERR_INVALID
    assert lib.iekv_noop(1, 0, None) == _native.IEKV_OK


def test_scattered_restore_rejects_missing_host_addresses(lib):
    """A slab pool registers without touching the GPU; the host address list is
    checked before anything is enqueued."""
    from iekv import _native

    pool = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    ids = (ctypes.c_int32 * 2)(0, 1)
    rc = lib.iekv_restore_blocks(pool.handle, ids, 2, None, None, 0, None, None)
    assert rc == _native.IEKV_ERR_INVALID
    assert "host block address list is null" in lib.iekv_last_error().decode()
    blocks = (ctypes.c_void_p * 2)(4096, None)
    rc = lib.iekv_restore_blocks(pool.handle, ids, 2, blocks, None, 0, None, None)
    assert rc == _native.IEKV_ERR_INVALID
    assert "host block 1 address is null" in lib.iekv_last_error().decode()
    pool.close()


def test_static_offload_refuses_blocks_larger_than_its_buffer(lib):
    """iekv_offload_static checks its arguments, and that one block image fits the
    library's static staging buffer, before anything touches the GPU."""
    from iekv import _native

    small = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    ids = (ctypes.c_int32 * 2)(0, 1)
    host = ctypes.create_string_buffer(2 * 2 * 64)
    assert lib.iekv_offload_static(None, ids, 2, host, len(host), None, None) == \
        _native.IEKV_ERR_INVALID
    assert lib.iekv_offload_static(small.handle, None, 2, host, len(host), None, None) == \
        _native.IEKV_ERR_INVALID
    rc = lib.iekv_offload_static(small.handle, ids, 2, host, len(host) - 1, None, None)
    assert rc == _native.IEKV_ERR_CAPACITY
    assert "host buffer" in lib.iekv_last_error().decode()
    small.close()
    # Two arrays of 17 MiB tiles: a 34 MiB block image, over the 32 MiB buffer.
    tile = 17 << 20
    big = _native.Pool([1 << 40, (1 << 40) + 4 * tile], tile_bytes=tile, num_blocks=4, device=0)
    rc = lib.iekv_offload_static(big.handle, ids, 1, host, 1 << 40, None, None)
    assert rc == _native.IEKV_ERR_CAPACITY
    message = lib.iekv_last_error().decode()
    assert f"{2 * tile}" in message and f"{_native.STATIC_STAGING}-byte static staging" in message
    big.close()


def test_a_failing_hip_call_surfaces_as_a_hip_error(lib):
    """A HIP runtime failure inside the library comes back as IEKV_ERR_HIP with the
    runtime's own message, and in Python as NativeError (a RuntimeError, the
    reference's failure type, ie/serve/disaggregated.py:78-79). Arrays that are not
    equally spaced need an address table on the device, so registering them on a
    device that does not exist makes the runtime refuse to switch to it."""
    from iekv import _native

    ptrs = [1 << 30, (1 << 30) + 4096, (1 << 30) + 3 * 4096]
    out = ctypes.c_void_p()
    table = (ctypes.c_uint64 * 3)(*ptrs)
    rc = lib.iekv_pool_create(table, 3, 64, 16, 99, ctypes.byref(out))
    assert rc == _native.IEKV_ERR_HIP
    message = lib.iekv_last_error().decode()
    assert message.startswith("cannot make device 99 current: ")
    assert len(message) > len("cannot make device 99 current: ")   # the runtime's text
    assert not out.value
    with pytest.raises(_native.NativeError) as err:
        _native.Pool(ptrs, tile_bytes=64, num_blocks=16, device=99)
    assert err.value.code == _native.IEKV_ERR_HIP
    assert isinstance(err.value, RuntimeError)


def test_default_launch_shape():
    """A fresh process starts with the shape the header documents."""
    import json
    import subprocess
    import sys

    code = ("import sys; sys.path[:0] = [sys.argv[1]]; import json; from iekv import _native; "
            "print(json.dumps(_native.get_launch()))")
    out = subprocess.run([sys.executable, "-c", code, str(ROOT / "inference-engine_amd")],
                         capture_output=True, text=True, check=True, timeout=120)
    assert json.loads(out.stdout.strip().splitlines()[-1]) == {
        "run_blocks": 0, "unroll": 8, "nontemporal": 1, "order": 5, "pack_order": 0,
        "chunk_bytes": 4096, "direct_chunk_bytes": 8192}


def test_launch_settings_are_validated(lib):
    from iekv import _native

    before = _native.get_launch()
    with pytest.raises(_native.NativeError):
        _native.set_launch(run_blocks=65)
    with pytest.raises(_native.NativeError):
        _native.set_launch(unroll=3)
    with pytest.raises(_native.NativeError):
        _native.set_launch(nontemporal=2)
    for bad in (8, 9, -2):
        with pytest.raises(_native.NativeError):
            _native.set_launch(order=bad)
        with pytest.raises(_native.NativeError):
            _native.set_launch(pack_order=bad)
    for bad in (-2, 32, 100, 3000, 1 << 21):
        with pytest.raises(_native.NativeError):
            _native.set_launch(chunk_bytes=bad)
        with pytest.raises(_native.NativeError):
            _native.set_launch(direct_chunk_bytes=bad)
    _native.set_launch(order=3, pack_order=7)
    assert (_native.get_launch()["order"], _native.get_launch()["pack_order"]) == (3, 7)
    _native.set_launch(run_blocks=8, unroll=16, nontemporal=0, order=6, pack_order=1,
                       chunk_bytes=1024)
    # chunk_bytes sets the pool-to-pool moves' chunk too.
    assert _native.get_launch() == {"run_blocks": 8, "unroll": 16, "nontemporal": 0, "order": 6,
                                    "pack_order": 1, "chunk_bytes": 1024,
                                    "direct_chunk_bytes": 1024}
    _native.set_launch(unroll=1, chunk_bytes=0)
    assert _native.get_launch()["unroll"] == 1 and _native.get_launch()["chunk_bytes"] == 0
    assert _native.get_launch()["direct_chunk_bytes"] == 0
    _native.set_launch(direct_chunk_bytes=16384)
    assert _native.get_launch()["chunk_bytes"] == 0
    assert _native.get_launch()["direct_chunk_bytes"] == 16384
    with pytest.raises(_native.NativeError):
        _native.call("iekv_get_direct_chunk", None)
    _native.set_launch(**before)
    assert _native.get_launch() == before


def test_the_product_refuses_cpu_caches():
    import torch

    from iekv.engine.copier import HipSlotCopier

    k = [torch.zeros(32, 2, 4)]
    with pytest.raises(ValueError, match="GPU caches"):
        HipSlotCopier(k, [t.clone() for t in k], 16)


def test_direct_copy_issue_order_keeps_every_pair():
    import numpy as np

    from iekv.engine.copier import issue_order

    rng = np.random.default_rng(3)
    src = rng.permutation(500)[:200]
    dst = rng.permutation(700)[:200]
    s, d = issue_order(src.tolist(), dst.tolist())
    assert list(d) == sorted(dst.tolist())
    assert sorted(zip(s.tolist(), d.tolist())) == sorted(zip(src.tolist(), dst.tolist()))
    with pytest.raises(ValueError):
        issue_order([1, 2], [3])


def test_the_header_is_plain_c_and_links_from_c(lib, tmp_path):
    """A C99 program includes include/iekv.h, links libiekv.so with gcc and calls it
    (no GPU needed): the boundary is usable from any C FFI (cgo, JNI, N-API, ctypes)."""
    import shutil
    import subprocess

    from iekv import _native

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not installed")
    source = tmp_path / "abi.c"
    source.write_text(
        '#include "iekv.h"\n'
        "#include <stdio.h>\n"
        "int main(void) {\n"
        "  if (iekv_abi_version() != IEKV_ABI_VERSION) return 1;\n"
        "  if (iekv_copy_direct(0, 0, 0, 0, 1, 0) != IEKV_ERR_INVALID) return 2;\n"
        "  if (iekv_copy_direct_ids(0, 0, 0, 0, IEKV_INLINE_IDS + 1, 0) != IEKV_ERR_INVALID)"
        " return 3;\n"
        '  printf("%d %d %lld %d %s\\n", IEKV_ABI_VERSION, IEKV_INLINE_IDS,\n'
        '         (long long)IEKV_HOST_DIRECT_MAX_BYTES, IEKV_INLINE_IMAGES,\n'
        '         iekv_last_error());\n'
        "  return 0;\n"
        "}\n")
    exe = tmp_path / "abi"
    libdir = _native.library_path().parent
    subprocess.run([gcc, "-std=c99", "-Wall", "-Werror", "-D__HIP_PLATFORM_AMD__",
                    f"-I{ROOT / 'include'}", "-I/opt/rocm/include", str(source),
                    f"-L{libdir}", "-liekv", f"-Wl,-rpath,{libdir}", "-o", str(exe)],
                   check=True, capture_output=True, timeout=120)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0, (out.returncode, out.stdout, out.stderr)
    version, inline_ids, direct_max, inline_images = out.stdout.split()[:4]
    assert int(inline_images) == _native.INLINE_IMAGES
    assert int(version) == lib.iekv_abi_version() == _native.ABI_VERSION
    assert int(inline_ids) == _native.INLINE_IDS      # the binding mirrors the header
    assert int(direct_max) == _native.HOST_DIRECT_MAX


def kernel_arguments(library) -> dict[str, tuple[int, list[str]]]:
    """(argument-segment bytes, argument kinds) of every gfx950 kernel in the
    library, read from the code object's metadata notes with the ROCm LLVM tools."""
    import shutil
    import subprocess
    import tempfile
    from pathlib import Path

    tools = Path("/opt/rocm/llvm/bin")
    needed = ["llvm-objcopy", "clang-offload-bundler", "llvm-readelf"]
    if not all((tools / t).exists() or shutil.which(t) for t in needed):
        pytest.skip("the ROCm LLVM tools are not installed")
    tool = {t: str(tools / t) if (tools / t).exists() else shutil.which(t) for t in needed}
    with tempfile.TemporaryDirectory() as tmp:
        bundle, code = Path(tmp) / "fatbin", Path(tmp) / "gfx950.co"
        subprocess.run([tool["llvm-objcopy"], f"--dump-section=.hip_fatbin={bundle}",
                        str(library), str(Path(tmp) / "stripped")], check=True, timeout=60)
        subprocess.run([tool["clang-offload-bundler"], "--unbundle", "--type=o",
                        f"--input={bundle}", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                        f"--output={code}"], check=True, timeout=60)
        notes = subprocess.run([tool["llvm-readelf"], "--notes", str(code)], check=True,
                               capture_output=True, text=True, timeout=60).stdout
    kernels = {}
    for entry in notes.split("\n  - ")[1:]:
        name = re.search(r"^\s*\.name:\s+(\S+)", entry, re.M)
        size = re.search(r"\.kernarg_segment_size:\s*(\d+)", entry)
        if name and size:
            kinds = re.findall(r"\.value_kind:\s+(\S+)", entry)
            kernels[name.group(1)] = (int(size.group(1)), kinds)
    return kernels


def test_kernel_arguments_stay_small(lib):
    """The runtime copies a launch's whole argument segment into device memory for
    every launch, and on slower hosts that copy is most of a small launch's host
    cost (about 0.4 us per KiB, plus 0.2 to 0.8 us when a kernel reads gridDim and
    so carries the runtime's 256-byte block of hidden arguments). No kernel of the
    library has hidden arguments; the move kernel with device ids takes 128 bytes,
    and the kernels with ids in their arguments come in two sizes, the smaller
    (for up to 64 words of ids) under 400 bytes."""
    from iekv import _native

    kernels = kernel_arguments(_native.library_path())
    assert len(kernels) > 100
    hidden = sorted(n for n, (_, kinds) in kernels.items()
                    if any(k.startswith("hidden_") for k in kinds))
    assert not hidden, hidden[:5]
    def sizes(tag):
        return {size for name, (size, _) in kernels.items() if tag in name}
    assert sizes("kv_move_inline")
    assert max(sizes("7kv_moveI")) <= 128
    small, large = sorted(sizes("kv_move_inline"))
    assert small < 400 and large > 2 * _native.INLINE_IDS * 4
    assert max(sizes("kv_scatter_rows") | sizes("kv_gather_rows")) <= 128


def test_a_missing_or_mismatched_library_fails_loudly(tmp_path):
    """There is no fallback: with IEKV_LIBRARY naming a file that does not exist, the
    first use of the library raises RuntimeError naming the path and how to build
    it; a library that exports every entry point but reports another ABI version
    is refused by that version. Each case runs in a child process of its own."""
    import os
    import shutil
    import subprocess
    import sys

    from iekv import _native

    probe = ("import sys\nsys.path.insert(0, {pkg!r})\nfrom iekv import _native\n"
             "try:\n    _native.lib()\n    print('loaded')\n"
             "except RuntimeError as e:\n    print('refused:', e)\n"
             ).format(pkg=str(ROOT / "inference-engine_amd"))

    def first_use(library):
        env = dict(os.environ, IEKV_LIBRARY=str(library))
        out = subprocess.run([sys.executable, "-c", probe], env=env, capture_output=True,
                             text=True, timeout=300)
        assert out.returncode == 0, out.stderr[-2000:]
        return out.stdout.strip()

    missing = tmp_path / "absent" / "libiekv.so"
    said = first_use(missing)
    assert said.startswith("refused:") and str(missing) in said and "build" in said
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc is not installed")
    stub = tmp_path / "stub.c"
    stub.write_text("".join(
        f"int {name}(void) {{ return {_native.ABI_VERSION - 1}; }}\n"
        if name == "iekv_abi_version" else f"int {name}(void) {{ return -1; }}\n"
        for name in _native.SIGNATURES))
    lib = tmp_path / "libiekv_stub.so"
    subprocess.run([gcc, "-shared", "-fPIC", str(stub), "-o", str(lib)], check=True,
                   capture_output=True, timeout=120)
    said = first_use(lib)
    assert said.startswith("refused:")
    assert f"ABI version {_native.ABI_VERSION - 1}, expected {_native.ABI_VERSION}" in said


def test_pool_shapes_devices_and_slot_ranges_are_checked_before_any_launch(lib):
    """Moves between pools of different tile layouts or devices, slot calls over
    layers or arrays the pool does not have or with a block size that does not
    divide the tile, and a timing session of no launches are each refused with
    IEKV_ERR_INVALID and a message naming the problem, before any HIP call (slab
    pools register without touching a GPU, whatever device they name)."""
    from iekv import _native

    a = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    b = _native.Pool([1 << 24, (1 << 24) + 128 * 16], tile_bytes=128, num_blocks=16, device=0)
    c = _native.Pool([1 << 28, (1 << 28) + 64 * 16], tile_bytes=64, num_blocks=16, device=1)
    ids = (ctypes.c_int32 * 2)(0, 1)
    counts = (ctypes.c_int32 * 1)(2)
    streams = (ctypes.c_void_p * 1)(None)
    slots = (ctypes.c_int64 * 2)(0, 1)
    rows = ctypes.create_string_buffer(4096)
    table = (ctypes.c_int32 * 2)(0, 1)

    def refused(code, *expect):
        assert code == _native.IEKV_ERR_INVALID, code
        message = lib.iekv_last_error().decode()
        assert all(e in message for e in expect), message

    for other, why in ((b, "differ in shape"), (c, "devices 0 and 1")):
        refused(lib.iekv_copy_direct(a.handle, other.handle, ids, ids, 2, None), why)
        refused(lib.iekv_copy_direct_ids(a.handle, other.handle, ids, ids, 2, None), why)
        refused(lib.iekv_copy_direct_requests(a.handle, other.handle, 1, counts, ids, ids,
                                              streams, 1, None), why)
    # a has one layer (a K and a V array) of 64-byte tiles
    refused(lib.iekv_write_slots_layers(a.handle, 0, 2, 4, rows, rows, 0, slots, 2, None),
            "layers 0..1 out of range for 1 layers")
    refused(lib.iekv_write_slots_layers(a.handle, 0, 1, 3, rows, rows, 0, slots, 2, None),
            "block_size 3 does not divide the 64-byte tile")
    refused(lib.iekv_gather_rows_arrays(a.handle, 1, 2, 4, table, 8, rows, len(rows), None),
            "arrays 1..2 out of range for 2 arrays")
    refused(lib.iekv_gather_rows_arrays(a.handle, 0, 2, 5, table, 8, rows, len(rows), None),
            "block_size 5 does not divide the 64-byte tile")
    for n in (0, (1 << 20) + 1):
        refused(lib.iekv_profile_start(n), f"max_launches {n} out of range")
    for pool in (a, b, c):
        pool.close()


def test_the_integration_guides_ctypes_stub_matches_the_abi():
    """The integration guide shows the ctypes binding a maintainer of the reference
    would add; every argument list it declares must be the one the library is bound
    with here (iekv._native.SIGNATURES, itself checked against include/iekv.h)."""
    from ctypes import POINTER, c_int32, c_int64, c_uint64, c_void_p

    from iekv import _native

    text = (ROOT / "INTEGRATION.md").read_text()
    aliases = {"u64p": POINTER(c_uint64), "vp": c_void_p, "i32": c_int32, "i64": c_int64,
               "ctypes.POINTER(vp)": POINTER(c_void_p), "ctypes.c_uint64": c_uint64}
    declared = re.findall(r"^lib\.(iekv_\w+)\.argtypes = \[([^\]]*)\]", text, re.M)
    assert len(declared) >= 5
    for name, args in declared:
        got = [aliases[a.strip()] for a in args.split(",")]
        want = _native.SIGNATURES[name][1]
        assert got == want, (name, got, want)
    assert "lib.iekv_last_error.restype = ctypes.c_char_p" in text


def test_request_queue_arguments_are_checked_before_any_hip_call(lib):
    """The request queue refuses, with IEKV_ERR_INVALID and a message, what it can tell
    is wrong without a GPU: a null handle or output, pools of other layouts, devices or
    overlapping memory, and idle / lifetime limits out of range; the calls on a queue
    refuse a null queue, and an empty submission needs no queue state at all. Nothing
    here reaches HIP (slab pools register without touching a GPU)."""
    from iekv import _native

    a = _native.Pool([1 << 20, (1 << 20) + 64 * 16], tile_bytes=64, num_blocks=16, device=0)
    b = _native.Pool([1 << 24, (1 << 24) + 128 * 16], tile_bytes=128, num_blocks=16, device=0)
    c = _native.Pool([1 << 28, (1 << 28) + 64 * 16], tile_bytes=64, num_blocks=16, device=1)
    # overlaps a without being the same pool: a's second array starts inside it
    d = _native.Pool([(1 << 20) + 64 * 8, 1 << 26], tile_bytes=64, num_blocks=16, device=0)
    out = ctypes.c_void_p()
    ticket = ctypes.c_uint64()
    flag = ctypes.c_int32()

    def refused(code, *expect):
        assert code == _native.IEKV_ERR_INVALID, code
        message = lib.iekv_last_error().decode()
        assert all(e in message for e in expect), message

    refused(lib.iekv_queue_create(a.handle, a.handle, 0, 0, 0, 0, None), "out is null")
    refused(lib.iekv_queue_create(None, a.handle, 0, 0, 0, 0, ctypes.byref(out)), "null")
    refused(lib.iekv_queue_create(a.handle, b.handle, 0, 0, 0, 0, ctypes.byref(out)),
            "differ in shape")
    refused(lib.iekv_queue_create(a.handle, c.handle, 0, 0, 0, 0, ctypes.byref(out)),
            "devices 0 and 1")
    refused(lib.iekv_queue_create(a.handle, d.handle, 0, 0, 0, 0, ctypes.byref(out)),
            "overlap")
    refused(lib.iekv_queue_create(a.handle, a.handle, -1, 0, 0, 0, ctypes.byref(out)),
            "negative")
    for idle, life in ((999, 0), (200_000, 300_000), (61_000_000, 0)):
        refused(lib.iekv_queue_create(a.handle, a.handle, 0, 0, idle, life, ctypes.byref(out)),
                "out of range")
    assert out.value is None
    ids = (ctypes.c_int32 * 1)(0)
    counts = (ctypes.c_int32 * 1)(1)
    tickets = (ctypes.c_uint64 * 1)()
    refused(lib.iekv_queue_submit(None, ids, ids, 1, ctypes.byref(ticket)), "queue is null")
    refused(lib.iekv_queue_submit_requests(None, 1, counts, ids, ids, tickets), "queue is null")
    refused(lib.iekv_queue_wait(None, 0, 0), "queue is null")
    refused(lib.iekv_queue_poll(None, 0, ctypes.byref(flag)), "null")
    refused(lib.iekv_queue_stop(None), "queue is null")
    refused(lib.iekv_queue_stats(None, None, None), "queue is null")
    assert lib.iekv_queue_destroy(None) == _native.IEKV_OK
