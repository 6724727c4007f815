"""mstar_amd -- the MI355X (gfx950) fused Mixture-of-Experts hot path.

Public surface (mirrors the reference's names):

* :mod:`mstar_amd.fused_moe` -- ``fused_experts``, ``moe_align_block_size``,
  ``moe_sum_reduce_triton``, ``act_and_mul_triton``,
  ``invoke_fused_moe_kernel``, ``get_default_config``.
* :mod:`mstar_amd.moe` -- ``TopKRouter``, ``SparseMoeBlock``,
  ``SparseMoeBlockWithSharedExpert``.
* :mod:`mstar_amd.linear` -- ``Fp8Linear``, ``fp8_scaled_mm``.
* :mod:`mstar_amd.quant` -- load-time weight quantisation.

All compute runs in ``libmstar_moe.so`` (hand-written HIP for gfx950, built
by :mod:`mstar_amd.build`); a missing library raises at first use.
"""
from __future__ import annotations

from ._lib import LIB_PATH, MstarError, load as load_library

__all__ = ["LIB_PATH", "MstarError", "load_library"]
