"""Fused router (mstar_moe_router): bf16 logits = hidden . Wg^T, fp32
softmax, top-k, renormalisation in one launch -- TopKRouter.forward
(mstar/model/components/moe.py:114-140).  The logits are checked against the
float64 closed form rounded to bf16 (within one bf16 rounding step: fp32
accumulation may round the other way at a boundary); the routing is checked
bit for bit against the oracle router applied to the kernel's own logits."""
from __future__ import annotations

import pytest
import torch

from oracle import moe_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run(M, H, E, k, renorm, seed):
    from mstar_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    wg = (torch.randn(E, H, generator=g) * 0.05).to(torch.bfloat16)
    xd, wd = x.to(DEV), wg.to(DEV)
    w = torch.empty(M, k, dtype=torch.float32, device=DEV)
    i32 = torch.empty(M, k, dtype=torch.int32, device=DEV)
    i64 = torch.empty(M, k, dtype=torch.int64, device=DEV)
    lg = torch.empty(M, E, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.mstar_moe_router(xd.data_ptr(), _lib.DT_BF16, M, H, wd.data_ptr(), E, k, int(renorm),
                                    w.data_ptr(), i32.data_ptr(), i64.data_ptr(), lg.data_ptr(),
                                    _lib.stream_of(xd)), "router")
    return x, wg, w.cpu(), i32.cpu(), i64.cpu(), lg.cpu()


@pytest.mark.parametrize("M,H,E,k,renorm", [(32, 2048, 128, 8, True), (1, 2048, 128, 8, True),
                                            (37, 256, 60, 4, False), (64, 256, 8, 2, True),
                                            (300, 1024, 256, 8, True), (17, 96, 200, 64, False)])
def test_router_vs_closed_form(M, H, E, k, renorm):
    x, wg, w, i32, i64, lg = _run(M, H, E, k, renorm, seed=M + E)
    exact = x.double() @ wg.double().t()
    ref = exact.to(torch.bfloat16).float()
    got = lg.float()
    # one bf16 step (2^-8 relative) covers fp32 accumulation rounding at a boundary
    assert torch.all((got - ref).abs() <= ref.abs() * 2.0 ** -7 + 1e-30)
    assert (got == ref).float().mean() > 0.99
    rw, rids = O.router_topk_softmax(got, k, renorm)
    assert torch.equal(i64, rids)
    assert torch.equal(i32.long(), rids)
    torch.testing.assert_close(w, rw, rtol=2e-6, atol=1e-9)


def test_router_module_and_errors():
    """mstar_amd.moe.TopKRouter uses the fused launch for bf16 and keeps the
    reference's 3-tuple contract; bad sizes are refused with a status."""
    from mstar_amd import _lib
    from mstar_amd.moe import TopKRouter
    r = TopKRouter(256, 16, 4).to(DEV).to(torch.bfloat16)
    with torch.no_grad():
        r.weight.copy_(torch.randn(16, 256, generator=torch.Generator().manual_seed(3)) * 0.05)
    x = torch.randn(2, 5, 256, generator=torch.Generator().manual_seed(4)).to(torch.bfloat16)
    w, ids, nxt = r(x.to(DEV))
    assert nxt is None and w.shape == (10, 4) and ids.dtype == torch.int64
    logits = (x.reshape(-1, 256).double() @ r.weight.detach().cpu().double().t()).to(torch.bfloat16)
    rw, rids = O.router_topk_softmax(logits.float(), 4, True)
    # ids from the closed-form logits match unless a bf16 rounding moved a near tie
    assert (ids.cpu() == rids).float().mean() > 0.95
    lib = _lib.load()
    assert lib.mstar_moe_router(None, _lib.DT_BF16, 4, 100, None, 8, 2, 1, None, None, None, None,
                                None) == 1  # H % 32 != 0
