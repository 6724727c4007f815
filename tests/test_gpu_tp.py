"""Tensor-parallel blocks on the GPU.

* One rank: ``ParallelSparseMoeBlock`` loaded through its weight loaders is
  ``SparseMoeBlock`` bit for bit (moe.py:446-450: world size 1 is the plain
  fused path).
* Two ranks on the one GPU (one process each, a gloo group carrying host
  copies): each rank holds half of every expert's intermediate size (bf16,
  then FP8 128x128 blocks), runs its shard through the fused layer and the
  group sums the partial outputs -- against the oracle of the full block,
  for the plain and the shared-expert block.  The reference's collective
  is an all-reduce over NCCL; RCCL would carry it on a multi-GPU node.
"""
from __future__ import annotations

import os
import socket
import subprocess
import sys

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
H, E, I, K_TOP = 1024, 32, 768, 4


def _checkpoint(seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(E, I, H, generator=g) * 0.02, torch.randn(E, I, H, generator=g) * 0.02,
            torch.randn(E, H, I, generator=g) * 0.02, torch.randn(E, H, generator=g) * 0.05)


def _load(blk, ckpt):
    gate, up, down, wg = ckpt
    ex = blk.experts
    for e in range(E):
        ex.gate_up_proj.weight_loader(ex.gate_up_proj, gate[e].to(ex.gate_up_proj.dtype).to(DEV), f"gate:{e}")
        ex.gate_up_proj.weight_loader(ex.gate_up_proj, up[e].to(ex.gate_up_proj.dtype).to(DEV), f"up:{e}")
        ex.down_proj.weight_loader(ex.down_proj, down[e].to(ex.down_proj.dtype).to(DEV), f"down:{e}")
    with torch.no_grad():
        blk.gate.weight.copy_(wg)


def test_one_rank_is_the_plain_block():
    from mstar_amd.moe import ParallelSparseMoeBlock, SparseMoeBlock
    ckpt = _checkpoint()
    p = ParallelSparseMoeBlock(H, E, K_TOP, I).to(DEV, torch.bfloat16)
    _load(p, ckpt)
    s = SparseMoeBlock(H, E, K_TOP, I).to(DEV, torch.bfloat16)
    with torch.no_grad():
        s.experts.gate_up_proj.copy_(p.experts.gate_up_proj)
        s.experts.down_proj.copy_(p.experts.down_proj)
        s.gate.weight.copy_(p.gate.weight)
    x = torch.randn(64, H, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16).to(DEV)
    assert torch.equal(p(x), s(x))


RANK = r'''
import os, sys, torch, torch.distributed as dist
from tests.test_gpu_tp import H, E, I, K_TOP, DEV, _checkpoint, _load
from mstar_amd.moe import ParallelSparseMoeBlock, ParallelSparseMoeBlockWithSharedExpert, ProcessGroupComm
rank, out_dir = int(os.environ["RANK"]), sys.argv[1]
dist.init_process_group("gloo", rank=rank, world_size=2)
comm = ProcessGroupComm()
ckpt = _checkpoint()
x = torch.randn(96, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16).to(DEV)
res = {}
for quant in (None, "fp8_w8a8"):
    blk = ParallelSparseMoeBlock(H, E, K_TOP, I, comm_group=comm).to(DEV, torch.bfloat16)
    _load(blk, ckpt)
    if quant:
        blk.quantize(quant)
    res[f"plain_{quant}"] = blk(x).cpu()
torch.manual_seed(3)
shared = torch.nn.Linear(H, H, bias=False)
sb = ParallelSparseMoeBlockWithSharedExpert(H, E, K_TOP, I, shared_expert=shared,
                                            comm_group=comm).to(DEV, torch.bfloat16)
_load(sb, ckpt)
res["shared"] = sb(x).cpu()
if rank == 0:
    torch.save(res, os.path.join(out_dir, "tp_out.pt"))
dist.destroy_process_group()
print(f"rank {rank} ok", flush=True)
'''


def test_two_ranks_sum_to_the_full_block(tmp_path):
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        port = s.getsockname()[1]
    env = dict(os.environ, MASTER_ADDR="127.0.0.1", MASTER_PORT=str(port), WORLD_SIZE="2",
               PYTHONPATH=REPO + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("two ranks on cuda:0 over gloo", flush=True)
    ps = [subprocess.Popen([sys.executable, "-c", RANK, str(tmp_path)], cwd=REPO,
                           env=dict(env, RANK=str(r)), stdout=subprocess.PIPE, stderr=subprocess.PIPE,
                           text=True) for r in range(2)]
    outs = [p.communicate(timeout=100) for p in ps]
    for p, (o, e) in zip(ps, outs):
        assert p.returncode == 0, o[-2000:] + e[-4000:]
    res = torch.load(str(tmp_path / "tp_out.pt"), weights_only=True)

    gate, up, down, wg = _checkpoint()
    x = torch.randn(96, H, generator=torch.Generator().manual_seed(2)).to(torch.bfloat16)
    wgb = wg.to(torch.bfloat16)
    logits = torch.nn.functional.linear(x.float(), wgb.float()).to(torch.bfloat16)
    w1 = torch.cat([gate, up], dim=1).to(torch.bfloat16)
    w2 = down.to(torch.bfloat16)
    tw, ti = O.router_topk_softmax(logits, K_TOP, True)
    half = I // 2
    sls = [slice(r * half, (r + 1) * half) for r in range(2)]

    def tp_sum(parts):
        # each rank stores its partial in bf16; the group sums those
        return (parts[0].float() + parts[1].float()).to(torch.bfloat16)

    def bf16_parts(tw_, ti_):
        return [O.fused_experts_rounding(x, torch.cat([gate[:, sl], up[:, sl]], 1).to(torch.bfloat16),
                                         down[:, :, sl].to(torch.bfloat16), tw_, ti_) for sl in sls]

    assert_moe_close(res["plain_None"], tp_sum(bf16_parts(tw, ti)), what="tp2 bf16 block")
    # and within bf16 noise of the unsharded block
    full = O.fused_experts_rounding(x, w1, w2, tw, ti)
    assert_moe_close(res["plain_None"], full, mean_of_rms=4e-3, what="tp2 bf16 vs unsharded")
    # FP8: blocks are local to each rank's slice, so dequantise per rank.
    from mstar_amd import quant as Q
    d1, d2 = [], []
    for sl in sls:
        q, s = Q.quantize_fp8_block(torch.cat([gate[:, sl], up[:, sl]], 1).to(torch.bfloat16))
        d1.append(O.dequant_fp8_block(q, s))
        q, s = Q.quantize_fp8_block(down[:, :, sl].to(torch.bfloat16))
        d2.append(O.dequant_fp8_block(q, s))
    parts = [O.fused_experts_rounding(x, None, None, tw, ti, w1_dq=d1[r], w2_dq=d2[r], act_quant=True)
             for r in range(2)]
    assert_moe_close(res["plain_fp8_w8a8"], tp_sum(parts), what="tp2 fp8 block")
    # Shared-expert block (norm_topk_prob False): the same construction
    # order rebuilds the shared expert and its gate from seed 3.
    from mstar_amd.moe import ParallelSparseMoeBlockWithSharedExpert
    torch.manual_seed(3)
    shared = torch.nn.Linear(H, H, bias=False)
    sb = ParallelSparseMoeBlockWithSharedExpert(H, E, K_TOP, I, shared_expert=shared)
    tw2, ti2 = O.router_topk_softmax(logits, K_TOP, False)
    routed = tp_sum(bf16_parts(tw2, ti2))
    sw = shared.weight.to(torch.bfloat16).float()
    gw = sb.shared_expert_gate.weight.to(torch.bfloat16).float()
    b = lambda t: t.to(torch.bfloat16).float()  # the block's eager bf16 rounding points
    ref3 = b(routed.float() + b(b(torch.sigmoid(b(x.float() @ gw.T))) * b(x.float() @ sw.T)))
    assert_moe_close(res["shared"], ref3, what="tp2 shared-expert block")
