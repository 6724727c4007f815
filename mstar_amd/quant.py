"""Weight quantisation at load time (FP8 block-scaled, FP8 per-channel, int4).

These run once when a checkpoint is loaded (the reference stacks expert
weights into ``gate_up_proj``/``down_proj`` at load, mstar/model/components/
moe.py:336-375), on whatever device the weight lives on, with PyTorch
tensor ops.  Formats (no reference counterpart -- the reference's quantised
branches were stripped, mstar/utils/fused_moe/kernels.py:3-7):

* FP8 block: one fp32 scale per 128x128 tile, ``s = max(amax, 1e-10)/448``,
  ``q = e4m3fn(clamp(w / s, -448, 448))`` (round to nearest even).  Both
  quotients are the correctly rounded fp32 values (computed in float64 and
  rounded once: PyTorch's GPU division by a scalar multiplies by the
  reciprocal, which can be one ulp off), so the codes do not depend on the
  device the weights are quantised on.
* FP8 per-channel: one scale per output row, same rule.
* int4 group-128: ``s = max(amax, 1e-10)/7`` rounded up to five significant
  bits (exact in bf16) per 128 of K, ``q = round(w / s)`` (within [-7, 7]),
  stored as ``u = q + 8`` nibbles, eight per int32, element ``k`` in bits
  ``4*(k % 8)`` of word ``k // 8``.  With five significant bits in ``s`` and
  at most three in ``q``, every dequantised weight ``q * s`` is exact in
  bf16, so a kernel may apply the scale after its dot products.
"""
from __future__ import annotations

import torch

FP8_MAX = 448.0
EPS = 1e-10


def _to_fp8(x: torch.Tensor) -> torch.Tensor:
    return x.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


def _div(a: torch.Tensor, b) -> torch.Tensor:
    """fp32 ``a / b`` correctly rounded on any device (float64 quotient of
    fp32 operands, rounded once)."""
    b = b.double() if torch.is_tensor(b) else float(b)
    return (a.double() / b).float()


def round_up_5bits(x: torch.Tensor) -> torch.Tensor:
    """Positive fp32 ``x`` rounded up to five significant bits (four mantissa
    bits): the smallest such value >= x."""
    bits = x.float().contiguous().view(torch.int32)
    step = 1 << (23 - 4)
    return ((bits + (step - 1)) & ~(step - 1)).view(torch.float32)


@torch.no_grad()
def quantize_fp8_block(w: torch.Tensor, block: tuple[int, int] = (128, 128)):
    """``w [..., N, K]`` -> ``(q e4m3fn [..., N, K], s fp32 [..., ceil(N/bn), ceil(K/bk)])``."""
    bn, bk = block
    *lead, N, K = w.shape
    nb, kb = -(-N // bn), -(-K // bk)
    if N % bn == 0 and K % bk == 0:
        wf = w.float()
    else:
        wf = torch.zeros(*lead, nb * bn, kb * bk, dtype=torch.float32, device=w.device)
        wf[..., :N, :K] = w.float()
    t = wf.view(*lead, nb, bn, kb, bk)
    s = _div(t.abs().amax(dim=(-3, -1)).clamp_min(EPS), FP8_MAX)
    q = _to_fp8(_div(t, s[..., :, None, :, None])).view(*lead, nb * bn, kb * bk)[..., :N, :K]
    return q.contiguous(), s.contiguous()


@torch.no_grad()
def quantize_fp8_per_channel(w: torch.Tensor):
    """``w [N, K]`` -> ``(q e4m3fn [N, K], s fp32 [N])``."""
    wf = w.float()
    s = _div(wf.abs().amax(dim=-1).clamp_min(EPS), FP8_MAX)
    return _to_fp8(_div(wf, s[..., None])).contiguous(), s.contiguous()


@torch.no_grad()
def quantize_int4_group(w: torch.Tensor, group: int = 128):
    """``w [..., N, K]`` -> ``(packed int32 [..., N, K/8], scales bf16 [..., N, K/group])``."""
    *lead, N, K = w.shape
    if K % group or K % 8:
        raise ValueError(f"quantize_int4_group: K={K} must be a multiple of {group} and 8")
    wf = w.float().view(*lead, N, K // group, group)
    s = round_up_5bits(_div(wf.abs().amax(dim=-1).clamp_min(EPS), 7.0)).to(torch.bfloat16)
    q = torch.round(_div(wf, s.float()[..., None])).clamp(-8, 7).to(torch.int32).view(*lead, N, K)
    u = (q + 8).view(*lead, N, K // 8, 8)
    packed = torch.zeros(*lead, N, K // 8, dtype=torch.int32, device=w.device)
    for i in range(8):
        packed |= u[..., i] << (4 * i)
    return packed.contiguous(), s.contiguous()


@torch.no_grad()
def dequantize_fp8_block(q: torch.Tensor, s: torch.Tensor, block=(128, 128)) -> torch.Tensor:
    bn, bk = block
    N, K = q.shape[-2], q.shape[-1]
    sf = s.repeat_interleave(bn, dim=-2)[..., :N, :].repeat_interleave(bk, dim=-1)[..., :K]
    return q.float() * sf


@torch.no_grad()
def dequantize_int4_group(packed: torch.Tensor, scales: torch.Tensor, group: int = 128) -> torch.Tensor:
    """-> bf16 ``q * s`` (the weight the W4A16 GEMM multiplies)."""
    p = packed.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, dtype=torch.int64, device=packed.device) * 4
    q = ((p[..., None] >> shifts) & 0xF) - 8
    q = q.reshape(*packed.shape[:-1], packed.shape[-1] * 8).float()
    return (q * scales.float().repeat_interleave(group, dim=-1)).to(torch.bfloat16)
