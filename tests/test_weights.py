"""FP8 weight loading (CPU): the per-expert, per-rank loaders equal the
block quantisation of the reference loaders' stacked bf16 parameters, and
the on-disk format round-trips."""
import os

import pytest
import torch

from mstar_amd import quant, weights


def _ref_stack(gate, up, down, tp_rank, tp_size):
    """The reference loaders' result (moe.py:335-375), restated: rank slice
    of the intermediate dimension, gate rows then up rows."""
    E, inter, H = gate.shape
    shard = inter // tp_size
    s0 = tp_rank * shard
    w1 = torch.cat([gate[:, s0:s0 + shard], up[:, s0:s0 + shard]], dim=1)
    w2 = down[:, :, s0:s0 + shard]
    return w1, w2


@pytest.mark.parametrize("tp_size", [1, 2])
def test_fp8_loaders_match_quantised_stack(tp_size):
    g = torch.Generator().manual_seed(0)
    E, H, inter = 3, 256, 512
    gate = (torch.randn(E, inter, H, generator=g) * 0.02).to(torch.bfloat16)
    up = (torch.randn(E, inter, H, generator=g) * 0.02).to(torch.bfloat16)
    down = (torch.randn(E, H, inter, generator=g) * 0.02).to(torch.bfloat16)
    for rank in range(tp_size):
        w1_q, w1_s, w2_q, w2_s = weights.empty_fp8_experts(E, H, inter, tp_size)
        for e in range(E):  # checkpoint order does not matter
            weights.fp8_down_proj_weight_loader(rank, tp_size, inter, w2_q, w2_s, down[e], f"down:{e}")
            weights.fp8_gate_up_weight_loader(rank, tp_size, inter, w1_q, w1_s, up[e], f"up:{e}")
            weights.fp8_gate_up_weight_loader(rank, tp_size, inter, w1_q, w1_s, gate[e], f"gate:{e}")
        w1, w2 = _ref_stack(gate, up, down, rank, tp_size)
        q1, s1 = quant.quantize_fp8_block(w1)
        q2, s2 = quant.quantize_fp8_block(w2)
        assert torch.equal(w1_q.view(torch.uint8), q1.view(torch.uint8)) and torch.equal(w1_s, s1)
        assert torch.equal(w2_q.view(torch.uint8), q2.view(torch.uint8)) and torch.equal(w2_s, s2)


def test_fp8_loader_rejects_unaligned_shards():
    with pytest.raises(ValueError):
        weights.empty_fp8_experts(2, 256, 384, tp_size=2)  # 192 per rank
    w = weights.empty_fp8_experts(1, 256, 256)
    with pytest.raises(ValueError):
        weights.fp8_gate_up_weight_loader(0, 1, 256, w[0], w[1], torch.zeros(256, 256), "mid:0")


def test_fp8_experts_round_trip(tmp_path):
    g = torch.Generator().manual_seed(1)
    w1_q, w1_s = quant.quantize_fp8_block(torch.randn(2, 256, 128, generator=g))
    w2_q, w2_s = quant.quantize_fp8_block(torch.randn(2, 128, 128, generator=g))
    p = os.path.join(tmp_path, "experts.safetensors")
    weights.save_fp8_experts(p, w1_q, w1_s, w2_q, w2_s)
    r = weights.load_fp8_experts(p)
    for a, b in zip(r, (w1_q, w1_s, w2_q, w2_s)):
        assert a.dtype == b.dtype and torch.equal(a.view(torch.uint8), b.view(torch.uint8))


def test_load_rejects_other_files(tmp_path):
    from safetensors.torch import save_file
    p = os.path.join(tmp_path, "other.safetensors")
    save_file({"x": torch.zeros(2)}, p)
    with pytest.raises(ValueError):
        weights.load_fp8_experts(p)
