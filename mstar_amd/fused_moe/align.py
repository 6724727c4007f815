"""Token-to-expert alignment (drop-in for mstar/utils/fused_moe/align.py:55-103).

``moe_align_block_size`` keeps the reference signature and output contract:
``sorted_token_ids`` (padding = ``topk_ids.numel()``), ``expert_ids`` (one per
``block_size`` block, unused blocks = 0) and ``num_tokens_post_padded`` (a
1-element device tensor, never read on the host).  It runs one HIP launch
(a single 1024-thread workgroup, deterministic: slots ascend within an
expert).  int32 and int64 ids are both accepted (the reference requires
int32, align.py:68).
"""
from __future__ import annotations

import torch

from .. import ops


def moe_align_block_size(topk_ids: torch.Tensor, block_size: int,
                         num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return ops.moe_align_block_size(topk_ids, block_size, num_experts)
