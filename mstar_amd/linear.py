"""Dense W8A8 FP8 linear (the FP8 replacement of the reference's ``F.linear``
in ColumnParallelLinear/RowParallelLinear/FusedColumnLinear,
mstar/model/components/distributed/linear.py:101,412 and
mstar/model/components/linear.py:94).

``y = bf16((A_q . W_q^T) * s_a[m] * s_w[n]) (+ bias)`` with per-token
activation scales (quantised inside :meth:`Fp8Linear.forward`) and
per-output-channel weight scales.
"""
from __future__ import annotations

import torch
from torch import nn

from . import ops, quant


def fp8_scaled_mm(a_q: torch.Tensor, a_scale: torch.Tensor, w_q: torch.Tensor,
                  w_scale: torch.Tensor) -> torch.Tensor:
    return ops.fp8_scaled_mm(a_q, a_scale, w_q, w_scale)


def fp8_linear(x: torch.Tensor, w_q: torch.Tensor, w_scale: torch.Tensor,
               bias: torch.Tensor | None = None) -> torch.Tensor:
    shape = x.shape
    a_q, a_s = ops.quant_fp8_per_token(x.reshape(-1, shape[-1]))
    y = ops.fp8_scaled_mm(a_q, a_s, w_q, w_scale)
    if bias is not None:
        y = y + bias
    return y.view(*shape[:-1], w_q.shape[0])


class Fp8Linear(nn.Module):
    def __init__(self, in_features: int, out_features: int, bias: bool = False,
                 device=None) -> None:
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.register_buffer("weight", torch.empty(out_features, in_features,
                                                   dtype=torch.float8_e4m3fn, device=device))
        self.register_buffer("weight_scale", torch.ones(out_features, dtype=torch.float32,
                                                        device=device))
        self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16, device=device)) if bias else None

    @classmethod
    def from_linear(cls, lin: nn.Linear) -> "Fp8Linear":
        m = cls(lin.in_features, lin.out_features, lin.bias is not None, device=lin.weight.device)
        q, s = quant.quantize_fp8_per_channel(lin.weight.data)
        m.weight.copy_(q)
        m.weight_scale.copy_(s)
        if lin.bias is not None:
            m.bias.data.copy_(lin.bias.data.to(torch.bfloat16))
        return m

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return fp8_linear(x, self.weight, self.weight_scale, self.bias)
