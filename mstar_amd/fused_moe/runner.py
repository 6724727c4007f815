"""Fused MoE entry point (drop-in for mstar/utils/fused_moe/runner.py:31-159).

``fused_experts`` keeps the reference's positional signature and contract
(bf16/fp16 activations, ``w1 [E, 2I, H]`` with rows ``[gate; up]``,
``w2 [E, H, I]``, any-int ``topk_ids``, ``reduce_results``) and adds
keyword-only quantisation arguments:

* ``quant="fp8_w8a8"``: ``w1``/``w2`` are ``float8_e4m3fn`` with fp32 block
  scales ``w1_scale [E, 2I/128, H/128]``, ``w2_scale [E, H/128, I/128]``
  (``block_shape=(128, 128)``); activations are quantised per token-group of
  128 inside the call.
* ``quant="w4a16"``: ``w1``/``w2`` are int32-packed int4
  (``[E, 2I, H/8]``/``[E, H, I/8]``) with bf16 group-128 scales
  (``[E, 2I, H/128]``/``[E, H, I/128]``); see :mod:`mstar_amd.quant`.

The whole computation (align, gate_up GEMM with fused activation, down GEMM
with the routed weight, top-k sum) is one C-ABI call; no host sync, static
output shapes, graph-capturable.
"""
from __future__ import annotations

from typing import Optional, Sequence

import torch

from .. import _lib, ops

_QUANT = {None: _lib.QUANT_NONE, "none": _lib.QUANT_NONE, "fp8_w8a8": _lib.QUANT_FP8_W8A8,
          "w4a16": _lib.QUANT_W4A16}


def fused_experts(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    activation: str = "silu",
    reduce_results: bool = True,
    *,
    quant: Optional[str] = None,
    w1_scale: Optional[torch.Tensor] = None,
    w2_scale: Optional[torch.Tensor] = None,
    block_shape: Optional[Sequence[int]] = None,
) -> torch.Tensor:
    """Grouped-GEMM MoE dispatch; returns ``[tokens, hidden]`` or, with
    ``reduce_results=False``, ``[tokens, top_k, hidden]`` (runner.py:155-156)."""
    assert hidden_states.is_contiguous(), "hidden_states must be contiguous"
    assert w1.is_contiguous(), "w1 must be contiguous"
    assert w2.is_contiguous(), "w2 must be contiguous"
    assert hidden_states.dim() == 2
    assert topk_weights.shape == topk_ids.shape
    if quant not in _QUANT:
        raise ValueError(f"fused_experts: unknown quant {quant!r}")
    q = _QUANT[quant]
    if q == _lib.QUANT_NONE:
        assert hidden_states.dtype in (torch.bfloat16, torch.float16)
        if w1.dtype != hidden_states.dtype or w2.dtype != hidden_states.dtype:
            raise ValueError("fused_experts: w1/w2 must match the hidden dtype when unquantised")
    else:
        if hidden_states.dtype != torch.bfloat16:
            raise ValueError(f"fused_experts: quant={quant} takes bf16 activations")
    if q == _lib.QUANT_FP8_W8A8:
        if block_shape is not None and tuple(block_shape) != (128, 128):
            raise ValueError("fused_experts: only block_shape=(128, 128) is supported")
        if w1.dtype != torch.float8_e4m3fn or w2.dtype != torch.float8_e4m3fn:
            raise ValueError("fused_experts: fp8_w8a8 weights must be float8_e4m3fn")
    if q == _lib.QUANT_W4A16 and (w1.dtype != torch.int32 or w2.dtype != torch.int32):
        raise ValueError("fused_experts: w4a16 weights must be int32-packed")
    if activation not in ("silu", "gelu"):
        raise ValueError(f"fused_experts: unsupported activation {activation!r}")
    return ops.fused_experts_op(hidden_states, w1, w2, topk_weights, topk_ids,
                                ops._act_code(activation), bool(reduce_results), q,
                                w1_scale, w2_scale)
