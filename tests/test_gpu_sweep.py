"""A seeded sweep of fused-layer shapes on the GPU, beyond the hand-picked
ones: random token counts, hidden and intermediate sizes, expert counts,
top-k, dtypes, routing skew and quantisation modes, through both
fused_experts and moe_layer, each against the oracle at the tolerance of
tests/_util.py (the routing ids bit-exactly).  The shapes are drawn once from
a fixed seed, so every run checks the same cases; each case's parameters are
in its test id."""
from __future__ import annotations

import random
import zlib

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _cases():
    rng = random.Random(20261202)
    cases = []
    for n in range(10):  # bf16 / fp16, any sizes
        E = rng.choice([2, 5, 8, 16, 60, 128, 160])
        cases.append(dict(quant=None, dtype=rng.choice(["bf16", "fp16"]),
                          M=rng.choice([1, 3, 17, 64, 100, 333, 700]),
                          H=rng.choice([32, 96, 136, 200, 256, 520, 1024]),
                          I=rng.choice([16, 48, 100, 128, 250, 384]),
                          E=E, k=rng.randint(1, min(8, E)), bias=rng.random() < 0.3, via="fused"))
    for n in range(8):  # FP8 W8A8, block 128
        E = rng.choice([8, 32, 64, 128, 256])
        cases.append(dict(quant="fp8_w8a8", dtype="bf16",
                          M=rng.choice([1, 5, 32, 64, 65, 200, 600, 1500]),
                          H=rng.choice([256, 512, 1024, 2048]), I=rng.choice([128, 256, 384, 768]),
                          E=E, k=rng.randint(1, min(8, E)), bias=rng.random() < 0.5,
                          via=rng.choice(["fused", "layer"])))
    for n in range(6):  # W4A16, group 128
        E = rng.choice([8, 32, 128])
        cases.append(dict(quant="w4a16", dtype="bf16", M=rng.choice([1, 8, 32, 100, 300]),
                          H=rng.choice([256, 512, 1024, 2048]), I=rng.choice([256, 512, 768]),
                          E=E, k=rng.randint(1, min(8, E)), bias=rng.random() < 0.5,
                          via=rng.choice(["fused", "layer"])))
    return cases


def _id(c):
    return (f"{c['quant'] or c['dtype']}-{c['via']}-M{c['M']}-H{c['H']}-I{c['I']}-E{c['E']}-k{c['k']}"
            + ("-zipf" if c["bias"] else ""))


CASES = _cases()


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_fused_layer_sweep(c):
    from mstar_amd import _lib, ops
    from mstar_amd import quant as Q
    from mstar_amd.fused_moe import fused_experts
    M, H, I, E, k = c["M"], c["H"], c["I"], c["E"], c["k"]
    dt = torch.bfloat16 if c["dtype"] == "bf16" else torch.float16
    seed = zlib.crc32(_id(c).encode()) % 10000
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(dt)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(dt)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(dt)
    logits = torch.randn(M, E, generator=g)
    if c["bias"]:
        logits = logits + O.zipf_bias(E)
    rw, rids = O.router_topk_softmax(logits, k, True)
    dq1 = dq2 = None
    if c["quant"] == "fp8_w8a8":
        q1, s1 = Q.quantize_fp8_block(w1.to(DEV))
        q2, s2 = Q.quantize_fp8_block(w2.to(DEV))
        c1, c2, c3, c4 = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
        dq1 = lambda e: O.dequant_fp8_block(c1[e], c2[e])
        dq2 = lambda e: O.dequant_fp8_block(c3[e], c4[e])
        code, kw = _lib.QUANT_FP8_W8A8, dict(quant="fp8_w8a8", block_shape=(128, 128))
    elif c["quant"] == "w4a16":
        q1, s1 = Q.quantize_int4_group(w1.to(DEV))
        q2, s2 = Q.quantize_int4_group(w2.to(DEV))
        c1, c2, c3, c4 = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
        dq1 = lambda e: O.dequant_int4_group(c1[e], c2[e])
        dq2 = lambda e: O.dequant_int4_group(c3[e], c4[e])
        code, kw = _lib.QUANT_W4A16, dict(quant="w4a16")
    else:
        q1, q2, s1, s2 = w1.to(DEV), w2.to(DEV), None, None
        code, kw = _lib.QUANT_NONE, {}
    print(f"sweep {_id(c)}", flush=True)
    if c["via"] == "layer":
        out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0, code, s1, s2)
        assert torch.equal(ti.cpu(), rids)
    else:
        out = fused_experts(x.to(DEV), q1, q2, rw.to(DEV), rids.to(DEV), w1_scale=s1, w2_scale=s2, **kw)
    ref = O.fused_experts_rounding(x, None if dq1 else w1, None if dq2 else w2, rw, rids,
                                   w1_dq=dq1, w2_dq=dq2, act_quant=c["quant"] == "fp8_w8a8")
    assert_moe_close(out, ref, what=f"sweep {_id(c)}")
