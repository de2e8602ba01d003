"""Host logic of sharded parameters (no GPU): where a DTensor's local shard
starts in the whole parameter, which the step uses to key its Philox
counters on the global element index (reference: optimizer.py:399-407 steps
the local shard of a DTensor; tests/test_fsdp.py:139-184 checks per-shard
scales).  Two CPU ranks over gloo, as FSDP2 shards parameters (Shard(0))."""

import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp
import torch.nn as nn

from luma_amd import LUMA
from luma_amd.optimizer import shard_offset


@pytest.mark.parametrize("backend", ["auto", "triton", "pytorch", "hip"])
def test_reference_backend_names_accepted(backend):
    """optimizer.py:98-113 accepts auto / triton / pytorch; every name selects HIP here."""
    assert LUMA(nn.Linear(4, 2).parameters(), backend=backend) is not None


def test_plain_tensor_offset_zero():
    assert shard_offset(torch.zeros(5, 3)) == 0


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


# shape, placement name, expected offset on rank 0 and rank 1 (world size 2)
CASES = [
    ((10, 6), "shard0", (0, 5 * 6)),
    ((4097,), "shard0", (0, 2049)),         # torch.chunk: 2049 + 2048 elements
    ((3, 8, 5), "shard0", (0, 2 * 8 * 5)),
    ((1, 12, 4), "shard1", (0, 6 * 4)),     # dims before the sharded one have extent 1
    ((10, 6), "shard1", (0, 0)),            # not one contiguous range: local keying
    ((10, 6), "replicate", (0, 0)),
]


def _rank_main(rank, world, port, out):
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        from torch.distributed.device_mesh import init_device_mesh
        from torch.distributed.tensor import Replicate, Shard, distribute_tensor
        mesh = init_device_mesh("cpu", (world,))
        res = []
        for shape, kind, _ in CASES:
            full = torch.arange(int(torch.tensor(shape).prod()), dtype=torch.float32).reshape(shape)
            pl = {"shard0": Shard(0), "shard1": Shard(1), "replicate": Replicate()}[kind]
            dt = distribute_tensor(full, mesh, [pl])
            off = shard_offset(dt)
            local = dt.to_local().contiguous().reshape(-1)
            # when the shard is one contiguous range, its elements are the
            # whole tensor's elements off, off + 1, ...
            contiguous = bool(torch.equal(local, full.reshape(-1)[off:off + local.numel()]))
            res.append((off, contiguous))
        out[rank] = res
    finally:
        dist.destroy_process_group()


def test_shard_offsets_two_ranks():
    mgr = mp.Manager()
    out = mgr.dict()
    mp.spawn(_rank_main, args=(2, _free_port(), out), nprocs=2, join=True)
    for i, (_, kind, want) in enumerate(CASES):
        for rank in range(2):
            off, contiguous = out[rank][i]
            assert off == want[rank], (CASES[i], rank, off)
            if kind != "shard1" or want[1] != 0:
                assert contiguous, (CASES[i], rank)
