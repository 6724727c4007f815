"""Fused MoE path on gfx950 (drop-in for ``mstar.utils.fused_moe``).

Exports the reference's public names (mstar/utils/fused_moe/__init__.py:14-17)
plus the alignment op.  Everything runs in hand-written HIP kernels from
``libmstar_moe.so``; there is no Triton and no CPU fallback.
"""
from __future__ import annotations

from .align import moe_align_block_size
from .kernels import (act_and_mul_triton, get_default_config, invoke_fused_moe_kernel,
                      moe_sum_reduce_triton)
from .runner import fused_experts

__all__ = ["fused_experts", "moe_sum_reduce_triton", "moe_align_block_size",
           "act_and_mul_triton", "invoke_fused_moe_kernel", "get_default_config"]
