"""Slot-level KV access on either side of the handoff, through libiekv.

``write_slots`` is the prefill side: it scatters a step's new K/V rows into the
pool by slot, as the reference's ``write_kv`` does (ie/kernels/reference.py:45-51,
ie/kernels/torch_backend.py:13-16). ``gather_rows`` is the decode side: it reads a
sequence's context back through its block table, as ``gather_context`` does
(ie/kernels/reference.py:54-63, ie/kernels/torch_backend.py:19-24). Slot
``r`` is row ``r`` of a layer's ``[N*bs, H, D]`` array, so both address the same
bytes the handoff moves.

``write_slots_layers`` and ``gather_rows_arrays`` do the same for many layers or
arrays in one launch: a forward pass's KV writes for every layer at once, and
a sequence's context in every layer's K and V cache at once.
"""
from __future__ import annotations

import torch

from .. import _native
from .pools import KVPool, current_stream_handle


def _device_slots(slots, device: torch.device) -> torch.Tensor:
    if isinstance(slots, torch.Tensor):
        t = slots.to(device=device, dtype=torch.int64)
    else:
        t = torch.as_tensor(slots, dtype=torch.int64, device=device)
    return t.contiguous()


def write_slots(pool: KVPool, layer: int, k: torch.Tensor, v: torch.Tensor, slots) -> None:
    """Scatter rows ``k[i]``, ``v[i]`` ([n, H, D]) into slot ``slots[i]`` of ``layer``.

    The rows are cast to the cache dtype first (as ``index_copy_`` of
    ``k.to(cache dtype)`` does); slots are range-checked on the host when given
    as a list.
    """
    n = k.shape[0]
    if v.shape[0] != n or len(slots) != n:
        raise ValueError(f"{len(slots)} slots for {n} K rows and {v.shape[0]} V rows")
    if tuple(k.shape[1:]) != pool.tile_shape[1:] or tuple(v.shape[1:]) != pool.tile_shape[1:]:
        raise ValueError(f"rows of shape {tuple(k.shape[1:])} do not fit a pool of "
                         f"{pool.tile_shape[1:]}")
    if not 0 <= layer < pool.num_layers:
        raise IndexError(f"layer {layer} out of range for {pool.num_layers} layers")
    if not isinstance(slots, torch.Tensor):
        rows = pool.num_blocks * pool.block_size
        bad = [s for s in slots if not 0 <= int(s) < rows]
        if bad:
            raise IndexError(f"slot {bad[0]} out of range for a pool of {rows} slots")
    kc = k.to(device=pool.device, dtype=pool.dtype).contiguous()
    vc = v.to(device=pool.device, dtype=pool.dtype).contiguous()
    st = _device_slots(slots, pool.device)
    stream = current_stream_handle(pool.device)
    _native.call("iekv_write_slots", pool.native.handle, layer, pool.block_size, kc.data_ptr(),
                 vc.data_ptr(), st.data_ptr(), n, stream)


def gather_rows(pool: KVPool, array: int, block_table, context_len: int) -> torch.Tensor:
    """Rows ``0..context_len-1`` of a sequence in array ``array`` (K of layer l is l, V is L+l).

    Returns a new ``[context_len, H, D]`` tensor of the cache dtype. Raises
    IndexError when the table is too short for ``context_len`` (as the
    reference does) or holds a block outside the pool.
    """
    bs = pool.block_size
    needed = -(-context_len // bs)
    if isinstance(block_table, torch.Tensor):
        table = block_table.to(dtype=torch.int32)
        if table.numel() < needed:
            raise IndexError(f"context of {context_len} needs {needed} blocks, table has "
                             f"{table.numel()}")
        table = table[:needed].to(pool.device).contiguous()
    else:
        if needed > len(block_table):
            raise IndexError(f"context of {context_len} needs {needed} blocks, table has "
                             f"{len(block_table)}")
        table = pool.block_ids(list(block_table[:needed]), what="context block")
    out = torch.empty((context_len, *pool.tile_shape[1:]), dtype=pool.dtype, device=pool.device)
    stream = current_stream_handle(pool.device)
    _native.call("iekv_gather_rows", pool.native.handle, array, bs, table.data_ptr(),
                 context_len, out.data_ptr(), out.numel() * out.element_size(),
                 stream)
    return out


def _check_slots(pool: KVPool, slots) -> None:
    if not isinstance(slots, torch.Tensor):
        rows = pool.num_blocks * pool.block_size
        bad = [s for s in slots if not 0 <= int(s) < rows]
        if bad:
            raise IndexError(f"slot {bad[0]} out of range for a pool of {rows} slots")


def write_slots_layers(pool: KVPool, k: torch.Tensor, v: torch.Tensor, slots,
                       first_layer: int = 0) -> None:
    """Scatter ``k[l, i]``, ``v[l, i]`` ([n_layers, n, H, D]) into slot ``slots[i]`` of
    layer ``first_layer + l``, every layer in one launch (rows cast to the cache dtype)."""
    if k.dim() != 4 or k.shape != v.shape:
        raise ValueError(f"K rows {tuple(k.shape)} and V rows {tuple(v.shape)} must both be "
                         "[n_layers, n, H, D]")
    n_layers, n = k.shape[0], k.shape[1]
    if len(slots) != n:
        raise ValueError(f"{len(slots)} slots for {n} rows per layer")
    if tuple(k.shape[2:]) != pool.tile_shape[1:]:
        raise ValueError(f"rows of shape {tuple(k.shape[2:])} do not fit a pool of "
                         f"{pool.tile_shape[1:]}")
    if first_layer < 0 or first_layer + n_layers > pool.num_layers:
        raise IndexError(f"layers {first_layer}..{first_layer + n_layers - 1} out of range for "
                         f"{pool.num_layers} layers")
    _check_slots(pool, slots)
    kc = k.to(device=pool.device, dtype=pool.dtype).contiguous()
    vc = v.to(device=pool.device, dtype=pool.dtype).contiguous()
    st = _device_slots(slots, pool.device)
    stride = n * kc.shape[2] * kc.shape[3] * kc.element_size()
    stream = current_stream_handle(pool.device)
    _native.call("iekv_write_slots_layers", pool.native.handle, first_layer, n_layers,
                 pool.block_size, kc.data_ptr(), vc.data_ptr(), stride, st.data_ptr(), n,
                 stream)


def gather_rows_arrays(pool: KVPool, block_table, context_len: int, first_array: int = 0,
                       n_arrays: int | None = None) -> torch.Tensor:
    """Rows ``0..context_len-1`` of a sequence in arrays ``first_array ..`` (all 2L by
    default: K of layers 0..L-1, then V), in one launch; a new
    ``[n_arrays, context_len, H, D]`` tensor of the cache dtype."""
    n_arrays = pool.n_arrays - first_array if n_arrays is None else n_arrays
    if first_array < 0 or n_arrays <= 0 or first_array + n_arrays > pool.n_arrays:
        raise IndexError(f"arrays {first_array}..{first_array + n_arrays - 1} out of range for "
                         f"{pool.n_arrays} arrays")
    bs = pool.block_size
    needed = -(-context_len // bs)
    if isinstance(block_table, torch.Tensor):
        table = block_table.to(dtype=torch.int32)
        if table.numel() < needed:
            raise IndexError(f"context of {context_len} needs {needed} blocks, table has "
                             f"{table.numel()}")
        table = table[:needed].to(pool.device).contiguous()
    else:
        if needed > len(block_table):
            raise IndexError(f"context of {context_len} needs {needed} blocks, table has "
                             f"{len(block_table)}")
        table = pool.block_ids(list(block_table[:needed]), what="context block")
    out = torch.empty((n_arrays, context_len, *pool.tile_shape[1:]), dtype=pool.dtype,
                      device=pool.device)
    stream = current_stream_handle(pool.device)
    _native.call("iekv_gather_rows_arrays", pool.native.handle, first_array, n_arrays, bs,
                 table.data_ptr(), context_len, out.data_ptr(), out.numel() * out.element_size(),
                 stream)
    return out
