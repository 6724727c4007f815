"""Any-shape 16-bit paths and the alignment extras on the GPU.

The reference's Triton kernel masks K and N tails (kernels.py:97-127 loads
with ``offs_k < K - k * BLOCK_SIZE_K``), so its unquantised fused_experts
accepts any hidden and intermediate size; these tests run the bf16 / fp16
layer and the reference runner's own call sequence at sizes that are not
multiples of 128 (nor of 8), against the oracle at the tolerance of
tests/_util.py.  The alignment's optional expert_offsets / expert_counts
are checked bit-exactly against the oracle's sorted_token_ids.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close
from tests.test_gpu_moe import _hidden, _routing, _weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("M,H,I,E,k,dtype", [
    (1, 32, 16, 8, 2, torch.bfloat16),
    (16, 32, 16, 8, 2, torch.bfloat16),
    (300, 32, 16, 8, 2, torch.bfloat16),
    (64, 200, 100, 8, 2, torch.bfloat16),     # K % 128 != 0; I % 8 != 0 (unaligned rows)
    (37, 33, 17, 4, 2, torch.bfloat16),       # odd H and I
    (130, 136, 72, 16, 4, torch.float16),
    (513, 130, 250, 8, 3, torch.float16),     # two 128-K steps, partial second
])
def test_fused_experts_any_shape(M, H, I, E, k, dtype):
    from mstar_amd.fused_moe import fused_experts
    w1, w2 = _weights(H, E, I, seed=H + I, dtype=dtype)
    x = _hidden(M, H, seed=M, dtype=dtype)
    tw, ti = _routing(M, E, k, seed=M + H)
    out = fused_experts(x.to(DEV), w1, w2, tw.to(DEV), ti.to(DEV))
    assert out.shape == (M, H) and out.dtype == dtype
    ref = O.fused_experts_rounding(x, w1.cpu(), w2.cpu(), tw, ti)
    assert_moe_close(out, ref, what=f"any-shape M={M} H={H} I={I} {dtype}")


@pytest.mark.parametrize("M,H,I", [(16, 33, 17), (300, 200, 100)])
def test_reference_composition_any_shape(M, H, I):
    """align -> GEMM1 -> act_and_mul -> GEMM2 -> sum-reduce
    (runner.py:99-159) at sizes off every vector width."""
    from mstar_amd.fused_moe import (act_and_mul_triton, get_default_config,
                                     invoke_fused_moe_kernel, moe_align_block_size,
                                     moe_sum_reduce_triton)
    E, k = 8, 2
    w1, w2 = _weights(H, E, I, seed=7)
    x = _hidden(M, H, seed=8).to(DEV)
    tw, ti = _routing(M, E, k, seed=9)
    tw_d, ti_d = tw.to(DEV), ti.to(DEV)
    cfg = get_default_config(M, E, 2 * I, H, k)
    s, e, n = moe_align_block_size(ti_d, cfg["BLOCK_SIZE_M"], E)
    c1 = torch.empty(M * k, 2 * I, dtype=torch.bfloat16, device=DEV)
    c2 = torch.empty(M * k, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(M, k, H, dtype=torch.bfloat16, device=DEV)
    invoke_fused_moe_kernel(x, w1, c1, tw_d, ti_d, s, e, n, False, k, cfg)
    act_and_mul_triton(c1, c2)
    invoke_fused_moe_kernel(c2, w2, c3.view(M * k, H), tw_d, ti_d, s, e, n, True, 1, cfg)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce_triton(c3, out)
    ref = O.fused_experts_rounding(x.cpu(), w1.cpu(), w2.cpu(), tw, ti)
    assert_moe_close(out, ref, what=f"composition any-shape M={M} H={H} I={I}")


@pytest.mark.parametrize("rows,inter", [(7, 13), (64, 100), (3, 1)])
def test_act_and_mul_tails(rows, inter):
    from mstar_amd.fused_moe import act_and_mul_triton
    g = torch.Generator().manual_seed(rows * inter)
    gu = torch.randn(rows, 2 * inter, generator=g).to(torch.bfloat16)
    out = torch.empty(rows, inter, dtype=torch.bfloat16, device=DEV)
    act_and_mul_triton(gu.to(DEV), out)
    ref = O.silu_and_mul_rounded(gu[:, :inter], gu[:, inter:])
    # At most one bf16 rounding step of the output and of act(gate) apart
    # (the device exponential is not torch's).
    diff = (out.cpu().float() - ref.float()).abs()
    ulp = ref.float().abs() * 2 ** -6 + 2.0 ** -133 * (1 + gu[:, inter:].float().abs())
    assert (diff <= ulp).all()


@pytest.mark.parametrize("tokens,k,hidden", [(5, 3, 33), (17, 8, 100)])
def test_sum_reduce_tails(tokens, k, hidden):
    from mstar_amd.fused_moe import moe_sum_reduce_triton
    g = torch.Generator().manual_seed(tokens * hidden)
    c3 = torch.randn(tokens, k, hidden, generator=g).to(torch.bfloat16)
    out = torch.empty(tokens, hidden, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce_triton(c3.to(DEV), out)
    ref = O.moe_sum_reduce(c3)
    diff = (out.cpu().float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2 ** -7 + 1e-30).all()


def _align_with_extras(ids: torch.Tensor, bs: int, E: int):
    from mstar_amd import _lib
    lib = _lib.load()
    numel = ids.numel()
    max_padded, max_blocks = O.align_sizes(numel, bs, E)
    d = ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=d)
    eids = torch.empty(max_blocks, dtype=torch.int32, device=d)
    ntpp = torch.empty(1, dtype=torch.int32, device=d)
    off = torch.full((E + 1,), -7, dtype=torch.int32, device=d)
    cnt = torch.full((E,), -7, dtype=torch.int32, device=d)
    nb = ctypes.c_size_t(0)
    _lib.check(lib.mstar_moe_align_scratch_size(numel, E, ctypes.byref(nb)), "scratch")
    scratch = torch.empty(max(nb.value, 4), dtype=torch.uint8, device=d)
    _lib.check(lib.mstar_moe_align_block_size(
        _lib.ptr(ids), _lib.dtype_code(ids.dtype), numel, E, bs, _lib.ptr(sorted_ids), max_padded,
        _lib.ptr(eids), max_blocks, _lib.ptr(ntpp), _lib.ptr(off), _lib.ptr(cnt), _lib.ptr(scratch),
        nb.value, _lib.stream_of(ids)), "align")
    torch.cuda.synchronize()
    return sorted_ids.cpu().numpy(), eids.cpu().numpy(), ntpp.cpu().numpy(), off.cpu().numpy(), cnt.cpu().numpy()


@pytest.mark.parametrize("M,E,k,bs,bias", [(1, 8, 2, 16, False), (64, 128, 8, 16, True),
                                           (700, 128, 8, 64, True), (4096, 64, 6, 256, False),
                                           (8192, 128, 8, 256, True)])
def test_align_expert_offsets_counts(M, E, k, bs, bias):
    """expert_offsets[e] is where expert e's padded run starts in the
    oracle's sorted_token_ids (offsets[E] = num_tokens_post_padded), and
    expert_counts[e] the real slots in that run -- read off the oracle's
    output, not restated from a formula.  Both the one-workgroup path
    (numel <= 4096) and the grid-wide path are covered."""
    _, ids = _routing(M, E, k, seed=M + E, bias=bias)
    sref, eref, nref = O.moe_align_block_size(ids.numpy(), bs, E)
    numel = ids.numel()
    for dt in (torch.int64, torch.int32):
        s, e, n, off, cnt = _align_with_extras(ids.to(dt).to(DEV), bs, E)
        assert np.array_equal(s, sref) and np.array_equal(e, eref) and np.array_equal(n, nref)
        ntpp = int(nref[0])
        assert off[0] == 0 and off[E] == ntpp
        for x in range(E):
            run = sref[off[x]:off[x + 1]]
            assert (off[x + 1] - off[x]) % bs == 0
            assert np.all(eref[off[x] // bs:off[x + 1] // bs] == x)
            assert cnt[x] == int(np.sum(run < numel))
            assert np.all(ids.reshape(-1).numpy()[run[run < numel]] == x)
        assert int(cnt.sum()) == numel
