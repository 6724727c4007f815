"""Kernel entry points of the fused MoE path (drop-in for
mstar/utils/fused_moe/kernels.py).

* :func:`invoke_fused_moe_kernel` -- grouped GEMM over expert-aligned blocks
  (kernels.py:141-218), backed by the gfx950 MFMA tile kernel.
* :func:`act_and_mul_triton` -- SwiGLU/GeGLU (kernels.py:279-298).
* :func:`moe_sum_reduce_triton` -- top-k sum (kernels.py:359-393).
* :func:`get_default_config` -- tile choice (kernels.py:401-420).

The ``*_triton`` names are kept so callers need no edits; no Triton is used.
"""
from __future__ import annotations

from typing import Any, Dict

import torch

from .. import ops


def get_default_config(M: int, E: int, N: int, K: int, top_k: int) -> Dict[str, int]:
    """Same result as the reference (kernels.py:401-420): the block size of
    the alignment step is 16 for decode-sized batches (M <= E), else 64."""
    if M <= E:
        return {"BLOCK_SIZE_M": 16, "BLOCK_SIZE_N": 32, "BLOCK_SIZE_K": 64, "GROUP_SIZE_M": 1}
    return {"BLOCK_SIZE_M": 64, "BLOCK_SIZE_N": 64, "BLOCK_SIZE_K": 32, "GROUP_SIZE_M": 8}


def invoke_fused_moe_kernel(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                            topk_weights: torch.Tensor, topk_ids: torch.Tensor,
                            sorted_token_ids: torch.Tensor, expert_ids: torch.Tensor,
                            num_tokens_post_padded: torch.Tensor, mul_routed_weight: bool,
                            top_k: int, config: Dict[str, Any], compute_type=None) -> None:
    """``C[slot] = A[slot // top_k] @ B[expert(slot)].T`` (times the routed
    weight when ``mul_routed_weight``), for bf16/fp16 operands; same
    arguments as the reference (kernels.py:141-154).  ``compute_type`` is
    accepted for signature compatibility; the output dtype is ``C.dtype``."""
    assert topk_weights.stride(1) == 1
    assert sorted_token_ids.stride(0) == 1
    if A.dtype != B.dtype or A.dtype != C.dtype:
        raise ValueError("invoke_fused_moe_kernel: A, B and C must share a dtype")
    ops.grouped_gemm(A, B, C.view(-1, C.shape[-1]), topk_weights, sorted_token_ids, expert_ids,
                     num_tokens_post_padded, topk_ids.numel(), top_k, mul_routed_weight,
                     config["BLOCK_SIZE_M"])


def act_and_mul_triton(gateup_output: torch.Tensor, down_input: torch.Tensor,
                       activation: str = "silu") -> None:
    """``down_input = act(gate) * up`` per row (kernels.py:279-298)."""
    ops.act_and_mul(gateup_output, down_input, ops._act_code(activation))


def moe_sum_reduce_triton(input: torch.Tensor, output: torch.Tensor,
                          routed_scaling_factor: float = 1.0) -> None:
    """``output = scale * input.sum(1)`` with fp32 accumulation (kernels.py:359-393)."""
    ops.moe_sum_reduce(input, output, float(routed_scaling_factor))


act_and_mul = act_and_mul_triton
moe_sum_reduce = moe_sum_reduce_triton
