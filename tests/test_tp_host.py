"""Host side of the tensor-parallel blocks (CPU, no GPU): the per-expert
weight loaders against a brute-force stacking of the checkpoint slices
(moe.py:335-375), and ProcessGroupComm's sum over a two-rank gloo group."""
from __future__ import annotations

import os
import socket

import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from mstar_amd.moe import ParallelSparseMoeBlock, ProcessGroupComm


class _Group:
    def __init__(self, rank, world_size):
        self.rank, self.world_size = rank, world_size

    def all_reduce(self, t):
        return t


@pytest.mark.parametrize("tp,rank", [(1, 0), (2, 0), (2, 1), (4, 3)])
def test_loaders_stack_the_rank_slices(tp, rank):
    H, E, I, k = 64, 4, 96, 2
    g = torch.Generator().manual_seed(tp * 10 + rank)
    gate = torch.randn(E, I, H, generator=g)
    up = torch.randn(E, I, H, generator=g)
    down = torch.randn(E, H, I, generator=g)
    blk = ParallelSparseMoeBlock(H, E, k, I, comm_group=_Group(rank, tp))
    assert blk.experts.gate_up_proj.shape == (E, 2 * I // tp, H)
    assert blk.experts.down_proj.shape == (E, H, I // tp)
    for e in range(E):
        blk.experts.gate_up_proj.weight_loader(blk.experts.gate_up_proj, gate[e], f"gate:{e}")
        blk.experts.gate_up_proj.weight_loader(blk.experts.gate_up_proj, up[e], f"up:{e}")
        blk.experts.down_proj.weight_loader(blk.experts.down_proj, down[e], f"down:{e}")
    s = I // tp
    rows = list(range(rank * s, (rank + 1) * s))
    for e in range(E):
        want1 = torch.stack([gate[e][r] for r in rows] + [up[e][r] for r in rows])
        want2 = torch.stack([down[e][:, c] for c in rows], dim=1)
        assert torch.equal(blk.experts.gate_up_proj.data[e], want1)
        assert torch.equal(blk.experts.down_proj.data[e], want2)
    blk = blk.to(torch.float64)  # loaders survive dtype / device moves
    assert blk.experts.down_proj.weight_loader.args == (rank, tp, I)


def test_loader_rejects_uneven_split():
    with pytest.raises(ValueError):
        ParallelSparseMoeBlock(64, 4, 2, 100, comm_group=_Group(0, 3))


def _worker(rank, world, port, q):
    os.environ.update(MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port))
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        c = ProcessGroupComm()
        t = torch.full((3, 5), float(rank + 1), dtype=torch.bfloat16)
        c.all_reduce(t)
        q.put((rank, c.rank, c.world_size, t.float().sum().item()))
    finally:
        dist.destroy_process_group()


def test_process_group_comm_sums_over_gloo():
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    ctx = mp.get_context("spawn")
    q = ctx.Queue()
    ps = [ctx.Process(target=_worker, args=(r, 2, port, q)) for r in range(2)]
    for p in ps:
        p.start()
    for p in ps:
        p.join(60)
        assert p.exitcode == 0
    got = sorted(q.get(timeout=5) for _ in range(2))
    assert got == [(0, 0, 2, 45.0), (1, 1, 2, 45.0)]
    assert ProcessGroupComm.trivial().world_size == 1
