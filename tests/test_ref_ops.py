"""The reference-named op ``torch.ops._mstar_moe_C.moe_align_block_size``
(mstar_amd/ref_ops.py), called the way the reference's align.py calls its
own extension: buffers allocated as align.py:78-87 does, outputs checked
bit-exactly against the oracle; errors raised as the reference op's
TORCH_CHECKs raise them (moe_align_block_size.cu:210-224)."""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O

# The schema text of moe_align_block_size.cu:273-277.
REFERENCE_SCHEMA = ("moe_align_block_size(Tensor topk_ids, int num_experts, int block_size, "
                    "Tensor! sorted_token_ids, Tensor! experts_ids, "
                    "Tensor! num_tokens_post_pad) -> ()")


def _op():
    from mstar_amd import ref_ops
    ref_ops.register()
    return torch.ops._mstar_moe_C.moe_align_block_size


def _reference_buffers(topk_ids, block_size, num_experts):
    """align.py:78-87: worst case one partial block padded per expert."""
    max_num_tokens_padded = topk_ids.numel() + num_experts * (block_size - 1)
    sorted_ids = torch.empty((max_num_tokens_padded,), dtype=torch.int32, device=topk_ids.device)
    max_num_m_blocks = math.ceil(max_num_tokens_padded / block_size)
    expert_ids = torch.empty((max_num_m_blocks,), dtype=torch.int32, device=topk_ids.device)
    ntpp = torch.empty((1,), dtype=torch.int32, device=topk_ids.device)
    return sorted_ids, expert_ids, ntpp


def test_schema_is_the_reference_schema():
    op = _op()
    from mstar_amd import ref_ops
    ref_ops.register()  # idempotent
    parsed = torch._C.parse_schema(f"{ref_ops.NAMESPACE}::{REFERENCE_SCHEMA}")
    got = op.default._schema
    assert got.name == parsed.name
    assert [a.name for a in got.arguments] == [a.name for a in parsed.arguments]
    assert [str(a.type) for a in got.arguments] == [str(a.type) for a in parsed.arguments]
    assert [bool(a.alias_info and a.alias_info.is_write) for a in got.arguments] == \
        [False, False, False, True, True, True]
    assert len(got.returns) == 0


def test_non_int32_ids_raise_runtime_error():
    op = _op()
    ids = torch.zeros(4, 2, dtype=torch.int64)
    s, e, n = _reference_buffers(ids, 16, 8)
    from mstar_amd.ref_ops import _align_impl
    with pytest.raises(RuntimeError, match="int32"):
        _align_impl(ids, 8, 16, s, e, n)


@pytest.mark.gpu
@pytest.mark.parametrize("M,E,k,zipf", [(32, 128, 8, False), (8192, 128, 8, True),
                                        (64, 8, 2, False), (1, 128, 8, False), (0, 128, 8, False)])
def test_reference_op_matches_oracle(M, E, k, zipf):
    op = _op()
    from mstar_amd.fused_moe import get_default_config
    block_size = get_default_config(M, E, 1536, 2048, k)["BLOCK_SIZE_M"]
    gen = torch.Generator().manual_seed(M + E)
    logits = torch.randn(M, E, generator=gen) + (O.zipf_bias(E) if zipf else 0)
    ids_cpu = torch.topk(logits, k).indices.to(torch.int32) if M else torch.zeros(0, k, dtype=torch.int32)
    ids = ids_cpu.cuda()
    s, e, n = _reference_buffers(ids, block_size, E)
    op(ids, E, block_size, s, e, n)
    torch.cuda.synchronize()
    rs, re, rn = O.moe_align_block_size(ids_cpu.numpy(), block_size, E)
    assert np.array_equal(s.cpu().numpy(), rs)
    assert np.array_equal(e.cpu().numpy(), re)
    assert np.array_equal(n.cpu().numpy(), rn)


@pytest.mark.gpu
def test_reference_op_rejects_1024_padded_experts():
    op = _op()
    E = 993  # rounded up to 32: 1024, which moe_align_block_size.cu:223 rejects
    ids = torch.zeros(4, 2, dtype=torch.int32, device="cuda")
    s, e, n = _reference_buffers(ids, 16, E)
    with pytest.raises(RuntimeError, match="1024"):
        op(ids, E, 16, s, e, n)
    with pytest.raises(RuntimeError, match="1024"):
        op(ids, 1024, 16, *_reference_buffers(ids, 16, 1024))
    # 992 experts (padded 992) is accepted.
    op(ids, 992, 16, *_reference_buffers(ids, 16, 992))
    torch.cuda.synchronize()


@pytest.mark.gpu
def test_reference_op_int64_ids_raise():
    op = _op()
    ids = torch.zeros(4, 2, dtype=torch.int64, device="cuda")
    with pytest.raises(RuntimeError, match="int32"):
        op(ids, 8, 16, *_reference_buffers(ids, 16, 8))
