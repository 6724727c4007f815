"""GPU parity: activation quantisation (bit-exact), dense FP8 scaled GEMM
(config 4), act_and_mul and the top-k sum-reduce."""
from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("rows,cols,scale", [(32, 2048, 1.0), (4096, 2048, 1.0), (7, 768, 30.0),
                                             (256, 128, 1e-3)])
def test_quant_fp8_per_token_group_bit_exact(rows, cols, scale):
    from mstar_amd import ops
    g = torch.Generator().manual_seed(rows)
    x = (torch.randn(rows, cols, generator=g) * scale).to(torch.bfloat16)
    x[0, :128] = 0
    q, s = ops.quant_fp8_per_token_group(x.to(DEV), 128)
    rq, rs = O.quant_fp8_per_token_group(x, 128)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


@pytest.mark.parametrize("rows,cols", [(32, 2048), (4096, 2048), (3, 100)])
def test_quant_fp8_per_token_bit_exact(rows, cols):
    from mstar_amd import ops
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(rows, cols, generator=g).to(torch.bfloat16)
    q, s = ops.quant_fp8_per_token(x.to(DEV))
    rq, rs = O.quant_fp8_per_row(x)
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)


def _dense(M, N, K, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    a = torch.randn(M, K, generator=g, device=DEV).to(torch.bfloat16)
    w = torch.randn(N, K, generator=g, device=DEV) * 0.02
    from mstar_amd import ops, quant
    aq, as_ = ops.quant_fp8_per_token(a)
    wq, ws = quant.quantize_fp8_per_channel(w)
    return aq, as_, wq, ws


@pytest.mark.parametrize("M,N", [(32, 4096), (32, 2048), (100, 2048), (4096, 4096),
                                 (65, 2048), (300, 1024)])  # row blocks with all-padding waves
def test_fp8_scaled_mm_vs_oracle(M, N):
    from mstar_amd import ops
    K = 2048
    aq, as_, wq, ws = _dense(M, N, K, seed=M + N)
    out = ops.fp8_scaled_mm(aq, as_, wq, ws)
    if M * N <= 32 * 4096 * 4:
        ref = O.fp8_scaled_mm(aq.cpu(), as_.cpu(), wq.cpu(), ws.cpu())
    else:  # large case: fp32 torch GEMM of the same FP8 codes on the GPU
        ref = ((aq.float() @ wq.float().T) * as_[:, None] * ws[None, :]).to(torch.bfloat16)
    assert_moe_close(out, ref, what=f"fp8_scaled_mm {M}x{N}")


@pytest.mark.parametrize("M,N,K", [(1, 4096, 2048), (7, 2064, 2048), (16, 2048, 256), (17, 4112, 1024),
                                   (32, 1040, 512)])
def test_fp8_scaled_mm_decode_stream(M, N, K):
    """M <= 32 runs the weight-streaming kernel: one and two token subtiles,
    channel counts that do not split evenly over the CUs, short K."""
    from mstar_amd import ops
    aq, as_, wq, ws = _dense(M, N, K, seed=M + N + K)
    out = ops.fp8_scaled_mm(aq, as_, wq, ws)
    ref = O.fp8_scaled_mm(aq.cpu(), as_.cpu(), wq.cpu(), ws.cpu())
    assert_moe_close(out, ref, what=f"fp8_scaled_mm stream {M}x{N}x{K}")


@pytest.mark.parametrize("M", [32, 4096])
def test_fp8_scaled_mm_lm_head(M):
    """N = 151936 (the vocabulary projection of config 4)."""
    from mstar_amd import ops
    aq, as_, wq, ws = _dense(M, 151936, 2048, seed=M)
    out = ops.fp8_scaled_mm(aq, as_, wq, ws)
    rows = slice(0, 8)
    ref = ((aq[rows].float() @ wq.float().T) * as_[rows, None] * ws[None, :]).to(torch.bfloat16)
    assert_moe_close(out[rows], ref, what="lm head rows")
    cols = torch.arange(0, 151936, 997, device=DEV)
    refc = ((aq.float() @ wq[cols].float().T) * as_[:, None] * ws[None, cols]).to(torch.bfloat16)
    assert_moe_close(out[:, cols], refc, what="lm head cols")


def test_fp8_linear_module():
    from mstar_amd.linear import Fp8Linear
    lin = torch.nn.Linear(2048, 512, bias=True).to(DEV, torch.bfloat16)
    m = Fp8Linear.from_linear(lin)
    x = torch.randn(4, 3, 2048, device=DEV, dtype=torch.bfloat16)
    with torch.no_grad():
        y = m(x)
        ref = lin(x).float()
    assert y.shape == (4, 3, 512)
    err = (y.float() - ref).abs().max() / ref.abs().max()
    assert float(err) < 0.06


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_act_and_mul_vs_oracle(dtype, act):
    from mstar_amd.fused_moe import act_and_mul_triton
    g = torch.Generator().manual_seed(1)
    gu = (torch.randn(257, 2 * 768, generator=g) * 3).to(dtype)
    out = torch.empty(257, 768, dtype=dtype, device=DEV)
    act_and_mul_triton(gu.to(DEV), out, activation=act)
    ref = O.silu_and_mul_rounded(gu[:, :768], gu[:, 768:], act)
    diff = (out.cpu().float() - ref.float()).abs()
    # One rounding step of the output plus one of the intermediate act(gate)
    # (scaled by |up|); the subnormal floor matters for fp16 gelu tails.
    rel = 2 ** -7 if dtype == torch.bfloat16 else 2 ** -10
    tiny = 2.0 ** -24 if dtype == torch.float16 else 2.0 ** -133
    up = gu[:, 768:].float().abs()
    ulp = ref.float().abs() * rel * 2 + tiny * (1 + up)
    assert (diff <= ulp).all()                # at most one rounding step apart
    assert (diff > 0).float().mean() < 0.01   # and almost always identical


def test_act_and_mul_matches_thread_device_case():
    # test/modular/test_worker_thread_device.py:45-80: all-ones input -> silu(1).
    from mstar_amd.fused_moe import act_and_mul_triton
    gu = torch.ones(4, 64, dtype=torch.bfloat16, device=DEV)
    out = torch.empty(4, 32, dtype=torch.bfloat16, device=DEV)
    act_and_mul_triton(gu, out)
    expect = torch.nn.functional.silu(torch.tensor(1.0)).to(torch.bfloat16)
    assert torch.equal(out.cpu(), torch.full((4, 32), float(expect), dtype=torch.bfloat16))


@pytest.mark.parametrize("T,k,H,scale", [(32, 8, 2048, 1.0), (8192, 8, 2048, 1.0), (5, 3, 24, 2.5)])
def test_sum_reduce_vs_oracle(T, k, H, scale):
    from mstar_amd.fused_moe import moe_sum_reduce_triton
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, k, H, generator=g).to(torch.bfloat16)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce_triton(x.to(DEV), out, scale)
    ref = O.moe_sum_reduce(x, scale)
    diff = (out.cpu().float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2 ** -7 + 1e-30).all()
