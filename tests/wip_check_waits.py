"""MSTAR_MOE_CHECK_WAITS=1: an eager moe_layer call whose one-launch decode
layer gave up a wait raises instead of returning NaN rows silently.  (Kept
out of collection until it has passed on the GPU.)"""
from __future__ import annotations

import pytest
import torch

from tests.test_gpu_layer_progress import layer_mode

pytestmark = pytest.mark.gpu


def test_check_waits_raises_on_give_up(monkeypatch):
    from mstar_amd import _lib, ops, quant
    E, H, I, k = 128, 2048, 768, 8
    g = torch.Generator().manual_seed(41)
    q1, s1 = quant.quantize_fp8_block((torch.randn(E, 2 * I, H, generator=g) * 0.02).cuda())
    q2, s2 = quant.quantize_fp8_block((torch.randn(E, H, I, generator=g) * 0.02).cuda())
    x = torch.randn(32, H, generator=g).to(torch.bfloat16).cuda()
    logits = torch.randn(32, E, generator=g).cuda()
    monkeypatch.setenv("MSTAR_MOE_CHECK_WAITS", "1")
    out, _, _ = ops.moe_layer(x, logits, q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)
    assert torch.isfinite(out.float()).all()
    with layer_mode(2):
        with pytest.raises(_lib.MstarError, match="gave up"):
            ops.moe_layer(x, logits, q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)
    out, _, _ = ops.moe_layer(x, logits, q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)
    assert torch.isfinite(out.float()).all()
