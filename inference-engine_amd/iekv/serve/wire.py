"""On-the-wire form of a KVTransfer, and point-to-point send / receive.

The reference's ``KVTransfer`` is an in-process Python object holding NumPy
payloads (ie/serve/disaggregated.py:16-25); prefill and decode never leave one
process. When they do (prefill GPU != decode GPU), a transfer travels as two
messages:

1. a self-describing header: magic ``b"IEKV"``, a little-endian u32 format
   version, a u32 length, then UTF-8 JSON with the sequence state
   (``token_ids``, ``num_computed``, ``first_block``, ``bytes_moved``) and the
   payload layout (blocks, layers, tile shape, dtype, tile bytes);
2. the payload itself: the block-major byte image ``[B, 2L, T]`` that
   ``iekv_pack`` writes (K tiles of layers 0..L-1, then V tiles, per block), so
   the receiver unpacks it with one ``iekv_unpack`` and nothing is re-laid-out.

``send_transfer`` / ``recv_transfer`` move both over ``torch.distributed``
point-to-point calls: a 2-int64 size message, the header bytes, then the payload
tensor. With the NCCL (RCCL) backend the tensors are device tensors and the
payload goes GPU to GPU over xGMI; with gloo they are host tensors.
"""
from __future__ import annotations

import json
import struct
from typing import Any

import torch

from .disaggregated import KVTransfer

MAGIC = b"IEKV"
WIRE_VERSION = 1
_PREFIX = struct.Struct("<4sII")   # magic, version, json length

_DTYPES = {
    "float32": torch.float32, "float16": torch.float16, "bfloat16": torch.bfloat16,
    "float8_e4m3fn": torch.float8_e4m3fn, "float8_e5m2": torch.float8_e5m2,
    "int8": torch.int8, "uint8": torch.uint8,
}
_NAMES = {v: k for k, v in _DTYPES.items()}


def _packed_of(transfer: KVTransfer):
    from ..engine.copier import BlockPayload, PackedBlocks, _consecutive_views, stack_payloads

    payloads = transfer.block_payloads
    if payloads is None:
        if transfer.source is None:
            raise ValueError("transfer carries neither payloads nor a source")
        packed = transfer.source.copier.read_blocks(transfer.source.block_ids)
        transfer.source.done()
        return packed
    if isinstance(payloads, PackedBlocks):
        return payloads
    items = list(payloads)
    view = _consecutive_views(items)
    if view is not None:
        return view
    if items and all(isinstance(p, BlockPayload) for p in items):
        return stack_payloads(items)     # rows of several buffers: gathered with one copy
    raise TypeError("wire transfers need PackedBlocks payloads (the HIP copier's)")


def encode_header(transfer: KVTransfer, packed) -> bytes:
    dtype = _NAMES.get(packed.dtype)
    if dtype is None:
        raise TypeError(f"no wire name for cache dtype {packed.dtype}")
    meta = {
        "token_ids": [int(t) for t in transfer.token_ids],
        "num_computed": int(transfer.num_computed),
        "first_block": int(transfer.first_block),
        "bytes_moved": int(transfer.bytes_moved),
        "num_blocks": len(packed),
        "num_layers": packed.num_layers,
        "tile_shape": list(packed.tile_shape),
        "dtype": dtype,
        "tile_bytes": packed.tile_bytes,
    }
    body = json.dumps(meta, separators=(",", ":")).encode()
    return _PREFIX.pack(MAGIC, WIRE_VERSION, len(body)) + body


def decode_header(buf: bytes) -> dict[str, Any]:
    if len(buf) < _PREFIX.size:
        raise ValueError("wire header is truncated")
    magic, version, length = _PREFIX.unpack_from(buf)
    if magic != MAGIC:
        raise ValueError(f"not a KV transfer header (magic {magic!r})")
    if version != WIRE_VERSION:
        raise ValueError(f"wire version {version} is not supported (expected {WIRE_VERSION})")
    body = bytes(buf[_PREFIX.size:_PREFIX.size + length])
    if len(body) != length:
        raise ValueError("wire header is truncated")
    meta = json.loads(body)
    if meta["dtype"] not in _DTYPES:
        raise ValueError(f"unknown cache dtype {meta['dtype']!r}")
    return meta


def to_wire(transfer: KVTransfer) -> tuple[bytes, torch.Tensor]:
    """(header bytes, payload tensor [B, 2L, T] uint8). Direct-mode transfers are packed first."""
    packed = _packed_of(transfer)
    # A host payload may still be filling from the device: hand out finished bytes.
    data = packed.host_data() if packed.on_host else packed.data
    return encode_header(transfer, packed), data


def from_wire(header: bytes, payload: torch.Tensor) -> KVTransfer:
    """Rebuild a KVTransfer whose payloads view ``payload`` (no copy)."""
    from ..engine.copier import PackedBlocks

    meta = decode_header(header)
    shape = (meta["num_blocks"], 2 * meta["num_layers"], meta["tile_bytes"])
    if payload.dtype != torch.uint8 or tuple(payload.shape) != shape:
        raise ValueError(f"payload of shape {tuple(payload.shape)} / {payload.dtype} does not "
                         f"match the header's {shape} uint8")
    packed = PackedBlocks(payload, meta["num_layers"], tuple(meta["tile_shape"]),
                          _DTYPES[meta["dtype"]])
    return KVTransfer(token_ids=list(meta["token_ids"]), num_computed=meta["num_computed"],
                      block_payloads=packed, bytes_moved=meta["bytes_moved"],
                      first_block=meta["first_block"])


def send_transfer(transfer: KVTransfer, dst: int, group=None,
                  device: torch.device | str | None = None) -> None:
    """Send a transfer to rank ``dst`` (blocking point-to-point calls)."""
    import torch.distributed as dist

    header, payload = to_wire(transfer)
    device = torch.device(device) if device is not None else payload.device
    sizes = torch.tensor([len(header), payload.numel()], dtype=torch.int64, device=device)
    dist.send(sizes, dst, group=group)
    dist.send(torch.frombuffer(bytearray(header), dtype=torch.uint8).to(device), dst, group=group)
    dist.send(payload.to(device).contiguous(), dst, group=group)


def recv_transfer(src: int, group=None, device: torch.device | str = "cpu") -> KVTransfer:
    """Receive a transfer sent by ``send_transfer`` from rank ``src`` into ``device`` memory."""
    import torch.distributed as dist

    device = torch.device(device)
    sizes = torch.empty(2, dtype=torch.int64, device=device)
    dist.recv(sizes, src, group=group)
    header_len, payload_len = (int(x) for x in sizes.tolist())
    header = torch.empty(header_len, dtype=torch.uint8, device=device)
    dist.recv(header, src, group=group)
    meta_bytes = header.cpu().numpy().tobytes()
    meta = decode_header(meta_bytes)
    shape = (meta["num_blocks"], 2 * meta["num_layers"], meta["tile_bytes"])
    if shape[0] * shape[1] * shape[2] != payload_len:
        raise ValueError("payload size does not match the header")
    payload = torch.empty(shape, dtype=torch.uint8, device=device)
    dist.recv(payload, src, group=group)
    return from_wire(meta_bytes, payload)
