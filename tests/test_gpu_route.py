"""GPU parity: softmax top-k routing and moe_align_block_size, bit-exact
against the oracle and the committed golden fixtures."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._util import align_brute_force

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
DEV = "cuda"


def _golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


@pytest.mark.parametrize("name,k,bm", [("route_tiny", 2, 64), ("route_decode", 8, 16),
                                       ("route_prefill512", 8, 64)])
def test_router_and_align_vs_golden(name, k, bm):
    from mstar_amd import ops
    g = _golden(name)
    logits = torch.from_numpy(g["logits"]).to(DEV)
    E = logits.shape[1]
    w, ids = ops.topk_softmax(logits, k, True)
    torch.cuda.synchronize()
    assert np.array_equal(ids.cpu().numpy(), g["topk_ids"])
    assert np.allclose(w.cpu().numpy(), g["topk_weights"], rtol=2e-6, atol=1e-9)
    s, e, n = ops.moe_align_block_size(ids, bm, E)
    assert np.array_equal(s.cpu().numpy(), g["sorted_token_ids"])
    assert np.array_equal(e.cpu().numpy(), g["expert_ids"])
    assert np.array_equal(n.cpu().numpy(), g["num_tokens_post_padded"])


@pytest.mark.parametrize("renorm", [True, False])
@pytest.mark.parametrize("M,E,k", [(1, 128, 8), (33, 128, 8), (100, 8, 2), (7, 60, 4),
                                   (5, 256, 8), (3, 1000, 16)])
def test_router_vs_oracle(M, E, k, renorm):
    from mstar_amd import ops
    gen = torch.Generator().manual_seed(M * 1000 + E)
    logits = torch.randn(M, E, generator=gen)
    w, ids = ops.topk_softmax(logits.to(DEV), k, renorm)
    rw, rids = O.router_topk_softmax(logits, k, renorm)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-9)


def test_router_bf16_logits_ties_take_lower_index():
    from mstar_amd import ops
    logits = torch.zeros(2, 16, dtype=torch.bfloat16)
    logits[0, [3, 5, 9]] = 1.0      # three-way tie at the top
    logits[1, :] = -2.0
    logits[1, 15] = 0.5
    w, ids = ops.topk_softmax(logits.to(DEV), 2, True)
    assert ids.cpu().tolist() == [[3, 5], [15, 0]]
    assert torch.allclose(w.cpu()[0], torch.tensor([0.5, 0.5]))


@pytest.mark.parametrize("shape,E,bm,dtype", [
    ((8192, 8), 128, 64, torch.int32),     # config 3 prefill, Zipf
    ((8192, 8), 128, 128, torch.int64),
    ((16384, 8), 128, 64, torch.int32),    # > 64k slots
    ((32, 8), 128, 16, torch.int64),
    ((1, 1), 1, 1, torch.int32),
    ((0, 8), 128, 16, torch.int32),        # empty
    ((40, 4), 16, 8, torch.int32),
    ((999, 3), 992, 32, torch.int32),      # largest expert count accepted
])
def test_align_vs_oracle(shape, E, bm, dtype):
    from mstar_amd import ops
    gen = torch.Generator().manual_seed(shape[0] + E)
    if shape[0] >= 8192:
        ids = torch.topk(torch.randn(shape[0], E, generator=gen) + O.zipf_bias(E), shape[1]).indices
    else:
        ids = torch.randint(0, E, shape, generator=gen)
    ids = ids.to(dtype)
    s, e, n = ops.moe_align_block_size(ids.to(DEV), bm, E)
    rs, re_, rn = O.moe_align_block_size(ids.numpy(), bm, E)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy(), re_)
    assert np.array_equal(n.cpu().numpy(), rn)


def test_align_skips_out_of_range_ids_like_reference():
    from mstar_amd import ops
    ids = torch.tensor([[0, 9], [3, 1], [8, 3]], dtype=torch.int32)  # 8, 9 >= E
    s, e, n = ops.moe_align_block_size(ids.to(DEV), 4, 8)
    bs, be, bn = align_brute_force(ids, 4, 8)
    assert s.cpu().tolist() == bs and e.cpu().tolist() == be and int(n.cpu()) == bn


def test_align_all_tokens_one_expert():
    from mstar_amd import ops
    ids = torch.full((4096, 8), 5, dtype=torch.int32)
    ids[:, 1:] = torch.arange(1, 8, dtype=torch.int32) + 10
    s, e, n = ops.moe_align_block_size(ids.to(DEV), 64, 128)
    rs, re_, rn = O.moe_align_block_size(ids.numpy(), 64, 128)
    assert np.array_equal(s.cpu().numpy(), rs) and np.array_equal(e.cpu().numpy(), re_)
    assert int(n.cpu()) == int(rn[0])


@pytest.mark.parametrize("M,E,k,bm,bias,dt", [
    (32, 128, 8, 16, False, torch.float32),      # decode: one launch
    (64, 128, 8, 32, True, torch.float32),       # exactly 512 slots: one launch
    (65, 128, 8, 32, True, torch.float32),       # 520 slots: grid path, one ragged block
    (512, 128, 8, 64, True, torch.float32),      # 4096 slots: grid path, 16 blocks
    (600, 128, 8, 64, True, torch.float32),      # grid path, ragged last block
    (8192, 128, 8, 64, True, torch.float32),     # config 3 prefill (32 tokens per workgroup)
    (5000, 128, 8, 64, True, torch.float32),     # 20 tokens per workgroup, ragged last block
    (1000, 64, 6, 32, False, torch.bfloat16),    # bf16 logits (ties), k=6
    (3, 8, 2, 64, False, torch.float32),
])
def test_route_fused_vs_oracle(M, E, k, bm, bias, dt):
    from mstar_amd import ops
    gen = torch.Generator().manual_seed(M + E + k)
    logits = torch.randn(M, E, generator=gen)
    if bias:
        logits = logits + O.zipf_bias(E)
    logits = logits.to(dt)
    w, ids, s, e, n = ops.moe_route(logits.to(DEV), k, True, bm)
    rw, rids = O.router_topk_softmax(logits.float(), k, True)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-9)
    rs, re_, rn = O.moe_align_block_size(rids.numpy(), bm, E)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy(), re_)
    assert np.array_equal(n.cpu().numpy(), rn)
