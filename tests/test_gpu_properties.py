"""Size-independent exact properties of the layer at BASELINE's full shapes
(H=2048, E=128, top-8, I=768), for FP8 W8A8, W4A16 and bf16 weights: decode
M=32 (the weight-streaming kernels), M=1024 (for FP8, the 128-row tile GEMM)
and prefill M=8192 with the Zipf bias (routing, alignment, the tile GEMMs,
the top-k sum).  Every row of the output
is checked, bit for bit, with no tolerance:

* routed weights times 2 -> output times 2: the routed weight enters only
  the down GEMM's fp32 epilogue and the fp32 top-k sum
  (kernels.py:129-133, 340-355), where scaling by a power of two commutes
  with every rounding;
* tokens permuted -> output rows permuted: each slot's arithmetic depends on
  its own token row and expert only, whatever position the alignment gives
  it (align.py:124-152 sorts slots by expert);
* experts relabelled (weights and routing permuted together) -> the same
  output: the expert order changes every block offset and position, not the
  arithmetic of any slot.

The dense W8A8 GEMM gets the matching checks over its whole output at the
LM-head shape.  The oracle comparisons of these paths are in test_gpu_moe.py
and test_gpu_dense_quant.py; these checks cover the rows and orderings that
those score only on a subset."""
from __future__ import annotations

import functools

import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, E, K_TOP, INTER = 2048, 128, 8, 768


@functools.lru_cache(maxsize=1)
def _bf16_weights():
    g = torch.Generator(device=DEV).manual_seed(21)
    w1 = (torch.randn(E, 2 * INTER, H, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    w2 = (torch.randn(E, H, INTER, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    return w1, w2


@functools.lru_cache(maxsize=3)
def _weights(quant):
    """(w1, w1_scale, w2, w2_scale) in the layout fused_experts takes."""
    from mstar_amd import quant as Q
    w1, w2 = _bf16_weights()
    if quant == "fp8_w8a8":
        q1, s1 = Q.quantize_fp8_block(w1)
        q2, s2 = Q.quantize_fp8_block(w2)
        return q1, s1, q2, s2
    if quant == "w4a16":
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        return q1, s1, q2, s2
    return w1, None, w2, None


def _inputs(M, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g)
    if M > 1024:
        logits = logits + O.zipf_bias(E)
    tw, ti = O.router_topk_softmax(logits, K_TOP, True)
    return x.to(DEV), tw.to(DEV), ti.to(DEV)


def _run(quant, x, tw, ti, weights=None):
    from mstar_amd.fused_moe import fused_experts
    q1, s1, q2, s2 = weights or _weights(quant)
    kw = {} if quant is None else {"quant": quant, "w1_scale": s1, "w2_scale": s2}
    return fused_experts(x, q1, q2, tw, ti, **kw)


def _bits(t):
    return t.view(torch.int16)


QUANTS = ["fp8_w8a8", "w4a16", None]


@pytest.mark.parametrize("quant", QUANTS, ids=["fp8", "w4a16", "bf16"])
@pytest.mark.parametrize("M", [32, 1024, 8192])
def test_routed_weight_scaling_is_exact(M, quant):
    x, tw, ti = _inputs(M, seed=M)
    print(f"properties: weight x2 M={M} {quant}", flush=True)
    base = _run(quant, x, tw, ti)
    doubled = _run(quant, x, tw * 2, ti)
    assert torch.isfinite(base.float()).all()
    assert torch.equal(_bits(doubled), _bits((base.float() * 2).to(torch.bfloat16)))


@pytest.mark.parametrize("quant", QUANTS, ids=["fp8", "w4a16", "bf16"])
@pytest.mark.parametrize("M", [32, 1024, 8192])
def test_token_permutation_is_exact(M, quant):
    x, tw, ti = _inputs(M, seed=M + 1)
    perm = torch.randperm(M, generator=torch.Generator().manual_seed(M)).to(DEV)
    print(f"properties: token permutation M={M} {quant}", flush=True)
    base = _run(quant, x, tw, ti)
    permuted = _run(quant, x[perm].contiguous(), tw[perm].contiguous(), ti[perm].contiguous())
    assert torch.equal(_bits(permuted), _bits(base[perm]))


@pytest.mark.parametrize("quant", QUANTS, ids=["fp8", "w4a16", "bf16"])
@pytest.mark.parametrize("M", [32, 1024, 8192])
def test_expert_relabelling_is_exact(M, quant):
    x, tw, ti = _inputs(M, seed=M + 2)
    q1, s1, q2, s2 = _weights(quant)
    # new expert e' = sigma(e): weights moved to their new index, ids mapped.
    sigma = torch.randperm(E, generator=torch.Generator().manual_seed(M + 2)).to(DEV)
    inv = torch.empty_like(sigma)
    inv[sigma] = torch.arange(E, device=DEV)
    relabelled = tuple(None if t is None else t[inv].contiguous() for t in (q1, s1, q2, s2))
    print(f"properties: expert relabelling M={M} {quant}", flush=True)
    base = _run(quant, x, tw, ti)
    moved = _run(quant, x, tw, sigma[ti].contiguous(), weights=relabelled)
    assert torch.equal(_bits(moved), _bits(base))


@pytest.mark.parametrize("M,N", [(4096, 151936), (32, 151936), (4096, 2048)])
def test_dense_fp8_properties_are_exact(M, N):
    """The dense W8A8 GEMM (y = bf16((A_q . W_q^T) s_a s_w)) over its whole
    output: permuting tokens and weight rows permutes the output's rows and
    columns, and doubling the per-channel scales doubles it."""
    from mstar_amd import ops, quant
    K = 2048
    g = torch.Generator(device=DEV).manual_seed(N + M)
    wq, ws = quant.quantize_fp8_per_channel(torch.randn(N, K, generator=g, device=DEV) * 0.02)
    aq, sa = ops.quant_fp8_per_token(torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16))
    print(f"properties: dense M={M} N={N}", flush=True)
    base = ops.fp8_scaled_mm(aq, sa, wq, ws)
    pm = torch.randperm(M, generator=torch.Generator().manual_seed(1)).to(DEV)
    pn = torch.randperm(N, generator=torch.Generator().manual_seed(2)).to(DEV)
    moved = ops.fp8_scaled_mm(aq[pm].contiguous(), sa[pm].contiguous(), wq[pn].contiguous(), ws[pn].contiguous())
    assert torch.equal(_bits(moved), _bits(base[pm][:, pn]))
    doubled = ops.fp8_scaled_mm(aq, sa, wq, ws * 2)
    assert torch.isfinite(base.float()).all()
    assert torch.equal(_bits(doubled), _bits((base.float() * 2).to(torch.bfloat16)))
