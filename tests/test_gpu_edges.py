"""Edge cases of the fused MoE path on the GPU: empty batches, top-1
routing, path boundaries (the 64-token streaming limit, 4096-slot routing
threshold), the tiny config 1 through the whole layer, and ragged
intermediate sizes -- each against the oracle at the tolerance of
tests/_util.py."""
from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close
from tests.test_gpu_moe import _fp8_ref, _fp8_weights, _hidden, _routing, _weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_empty_batches():
    """Zero tokens: every entry returns empty outputs without launching."""
    from mstar_amd import _lib, ops
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 256, 8, 256, 2
    w1, w2 = _weights(H, E, I)
    x = torch.empty(0, H, dtype=torch.bfloat16, device=DEV)
    ids = torch.empty(0, k, dtype=torch.int64, device=DEV)
    tw = torch.empty(0, k, dtype=torch.float32, device=DEV)
    assert fused_experts(x, w1, w2, tw, ids).shape == (0, H)
    out, w, i = ops.moe_layer(x, torch.empty(0, E, device=DEV), w1, w2, k, True, 0, _lib.QUANT_NONE,
                              None, None)
    assert out.shape == (0, H) and w.shape == (0, k) and i.shape == (0, k)
    w, i = ops.router(x, torch.zeros(E, H, dtype=torch.bfloat16, device=DEV), k, True)
    assert w.shape == (0, k)


@pytest.mark.parametrize("M", [64, 65, 513])
def test_fp8_path_boundaries(M):
    """64 tokens is the last weight-streaming batch, 65 the first tiled one;
    513 tokens x 8 is just past the single-workgroup routing limit."""
    from mstar_amd import _lib, ops
    H, E, I, k = 2048, 128, 768, 8
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = _hidden(M, H, seed=M + 5)
    g = torch.Generator().manual_seed(M + 6)
    logits = torch.randn(M, E, generator=g)
    rw, rids = O.router_topk_softmax(logits, k, True)
    out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8,
                                s1, s2)
    assert torch.equal(ti.cpu(), rids)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, rw, rids), what=f"fp8 boundary M={M}")


@pytest.mark.parametrize("M", [1, 32])
def test_fp8_top1(M):
    """top_k = 1 (every token to one expert) through the router-ids kernels."""
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 1
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = _hidden(M, H, seed=M + 7)
    tw, ti = _routing(M, E, k, seed=M + 7)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, tw, ti), what=f"fp8 top-1 M={M}")


def test_config1_layer_fp8():
    """Config 1 (M=64, H=256, E=8, top-2, I=512) through mstar_moe_layer."""
    from mstar_amd import _lib, ops
    M, H, E, I, k = 64, 256, 8, 512, 2
    q1, s1, q2, s2 = _fp8_weights(H, E, I, seed=1)
    x = _hidden(M, H, seed=41)
    logits = torch.randn(M, E, generator=torch.Generator().manual_seed(42))
    rw, rids = O.router_topk_softmax(logits, k, True)
    out, _, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8,
                               s1, s2)
    assert torch.equal(ti.cpu(), rids)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, rw, rids), what="config 1 fp8")


@pytest.mark.parametrize("I", [384, 640])
def test_fp8_ragged_intermediate(I):
    """Intermediate sizes that are multiples of 128 but not of 256 (the
    256-row prefill tile and the int4 decode chunks need care there)."""
    from mstar_amd.fused_moe import fused_experts
    H, E, k = 512, 16, 4
    q1, s1, q2, s2 = _fp8_weights(H, E, I, seed=2)
    for M in (16, 2048):
        x = _hidden(M, H, seed=M + I)
        tw, ti = _routing(M, E, k, seed=M + I)
        out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                            w1_scale=s1, w2_scale=s2)
        assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, tw, ti), what=f"fp8 I={I} M={M}")
