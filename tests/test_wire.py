"""KVTransfer wire format and point-to-point transport (CPU; gloo for the two-rank case)."""
from __future__ import annotations

import os
import socket

import numpy as np
import pytest
import torch

from oracle.copier import LayeredSlotCopier, pack, packed_image


def packed_from_oracle(layers=3, bs=4, heads=2, dim=8, blocks=(5, 1, 7), seed=0):
    """A transfer's payload built by the oracle, as the block-major image PackedBlocks holds."""
    from iekv.engine.copier import PackedBlocks

    rng = np.random.default_rng(seed)
    shape = (10 * bs, heads, dim)
    k = [rng.standard_normal(shape).astype(np.float32) for _ in range(layers)]
    v = [rng.standard_normal(shape).astype(np.float32) for _ in range(layers)]
    oracle = LayeredSlotCopier(k, v, bs)
    image = packed_image(pack(oracle, list(blocks)))
    packed = PackedBlocks(torch.from_numpy(image.copy()), layers, (bs, heads, dim), torch.float32)
    return packed, (k, v)


def make_transfer(packed):
    from iekv.serve.disaggregated import KVTransfer

    return KVTransfer(token_ids=list(range(100, 131)), num_computed=30, block_payloads=packed,
                      bytes_moved=packed.nbytes, first_block=2)


def test_round_trip_keeps_state_and_bytes():
    from iekv.serve.wire import from_wire, to_wire

    packed, _ = packed_from_oracle()
    transfer = make_transfer(packed)
    header, payload = to_wire(transfer)
    assert header[:4] == b"IEKV"
    back = from_wire(header, payload.clone())
    assert back.token_ids == transfer.token_ids
    assert back.num_computed == 30 and back.first_block == 2
    assert back.bytes_moved == transfer.bytes_moved
    assert back.num_blocks == 3 and back.table_length == 5
    assert torch.equal(back.block_payloads.data, packed.data)
    k_tiles, v_tiles = back.block_payloads[1]
    assert k_tiles[0].shape == (4, 2, 8) and k_tiles[0].dtype == torch.float32


def test_payloads_of_several_buffers_and_strided_slices_go_on_the_wire():
    """A transfer whose payload list mixes rows of two buffers, or takes every other
    row of one (both fine for the reference's list of payloads), goes on the wire
    as the rows in list order, gathered with one copy; the receiver's payloads are
    those rows. A list of something other than payloads is refused."""
    from iekv.serve.wire import from_wire, to_wire

    a, _ = packed_from_oracle(blocks=(5, 1, 7), seed=1)
    b, _ = packed_from_oracle(blocks=(2, 3), seed=2)
    for payloads, rows in (([a[2], b[0], a[0]], [a.data[2], b.data[0], a.data[0]]),
                           (a[::2], [a.data[0], a.data[2]]),
                           ([a[::2][1], b[1]], [a.data[2], b.data[1]])):
        transfer = make_transfer(a)
        transfer.block_payloads = payloads
        header, payload = to_wire(transfer)
        back = from_wire(header, payload.contiguous().clone())
        assert torch.equal(back.block_payloads.data, torch.stack(rows))
    transfer = make_transfer(a)
    transfer.block_payloads = [([np.zeros(4)], [np.zeros(4)])]
    with pytest.raises(TypeError):
        to_wire(transfer)


def test_payload_tiles_are_the_reference_payload():
    from iekv.serve.wire import from_wire, to_wire

    packed, (k, v) = packed_from_oracle(blocks=(9, 0))
    back = from_wire(*to_wire(make_transfer(packed)))
    k_tiles, v_tiles = back.block_payloads[0]
    for l in range(3):
        assert np.array_equal(k_tiles[l].numpy(), k[l][36:40])
        assert np.array_equal(v_tiles[l].numpy(), v[l][36:40])


@pytest.mark.parametrize("corrupt", ["magic", "version", "truncated", "shape"])
def test_bad_messages_are_rejected(corrupt):
    from iekv.serve.wire import from_wire, to_wire

    packed, _ = packed_from_oracle()
    header, payload = to_wire(make_transfer(packed))
    if corrupt == "magic":
        header = b"XXXX" + header[4:]
    elif corrupt == "version":
        header = header[:4] + (99).to_bytes(4, "little") + header[8:]
    elif corrupt == "truncated":
        header = header[:-3]
    else:
        payload = payload[:-1]
    with pytest.raises(ValueError):
        from_wire(header, payload)


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _rank_main(rank: int, port: int, result_path: str) -> None:
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    sys.path[:0] = [root, os.path.join(root, "inference-engine_amd"), os.path.dirname(__file__)]
    import torch.distributed as dist

    from iekv.serve.wire import recv_transfer, send_transfer

    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=2)
    try:
        packed, _ = packed_from_oracle(seed=11)
        if rank == 0:
            send_transfer(make_transfer(packed), dst=1)
        else:
            got = recv_transfer(src=0)
            ok = (torch.equal(got.block_payloads.data, packed.data)
                  and got.token_ids == list(range(100, 131)) and got.first_block == 2)
            with open(result_path, "w") as f:
                f.write("ok" if ok else "mismatch")
    finally:
        dist.destroy_process_group()


def test_send_and_receive_between_two_ranks(tmp_path):
    import torch.multiprocessing as mp

    result = tmp_path / "result.txt"
    mp.spawn(_rank_main, args=(_free_port(), str(result)), nprocs=2, join=True)
    assert result.read_text() == "ok"
