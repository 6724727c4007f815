"""The MoE block from hidden states, on the GPU.

* ``mstar_moe_block`` (fused router + experts in one library call, the path
  ``SparseMoeBlock.routed`` takes for bf16 states) against the oracle, with
  the routing read off the router kernel's own bf16 logits;
* fp16 blocks (``SparseMoeBlock`` and ``TopKRouter``: F.linear in fp16, then
  the HIP routing on fp16 logits);
* a layer run from FP8 experts quantised by ``mstar_amd.weights`` loaders,
  saved to safetensors and loaded back (moe.py:335-375's load-time stacking);
* W4A16 on plain bf16 ``amax / 7`` group scales (the common GPTQ form, no
  restriction on the scale's mantissa) against an exact dequantisation;
* argument checks of the public ops, which raise before any launch.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close
from tests.test_gpu_moe import _fp8_ref, _fp8_weights, _hidden, _routing, _weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _router_logits(x, wg):
    """The fused router's own bf16 logits (mstar_moe_router's logits_out)."""
    from mstar_amd import _lib
    M, H = x.shape
    E = wg.shape[0]
    lo = torch.empty(M, E, dtype=torch.bfloat16, device=DEV)
    w = torch.empty(M, 1, dtype=torch.float32, device=DEV)
    ids = torch.empty(M, 1, dtype=torch.int64, device=DEV)
    lib = _lib.load()
    _lib.check(lib.mstar_moe_router(_lib.ptr(x), _lib.DT_BF16, M, H, _lib.ptr(wg), E, 1, 1,
                                    _lib.ptr(w), None, _lib.ptr(ids), _lib.ptr(lo),
                                    _lib.stream_of(x)), "router")
    torch.cuda.synchronize()
    return lo.cpu()


@pytest.mark.parametrize("M,quant", [(1, "fp8_w8a8"), (32, "fp8_w8a8"), (700, "fp8_w8a8"),
                                     (32, None), (300, None), (32, "w4a16")])
def test_moe_block_one_call(M, quant):
    from mstar_amd import _lib, ops
    from mstar_amd import quant as Q
    H, E, I, k = 2048, 128, 768, 8
    x = _hidden(M, H, seed=M + 51).to(DEV)
    wg = (torch.randn(E, H, generator=torch.Generator().manual_seed(M)) * 0.05).to(torch.bfloat16).to(DEV)
    logits = _router_logits(x, wg)
    rw, rids = O.router_topk_softmax(logits, k, True)
    if quant == "fp8_w8a8":
        q1, s1, q2, s2 = _fp8_weights(H, E, I)
        code = _lib.QUANT_FP8_W8A8
        ref = _fp8_ref(x.cpu(), q1, s1, q2, s2, rw, rids)
    elif quant == "w4a16":
        w1, w2 = _weights(H, E, I)
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        code = _lib.QUANT_W4A16
        c = [t.cpu() for t in (q1, s1, q2, s2)]
        ref = O.fused_experts_rounding(x.cpu(), None, None, rw, rids,
                                       w1_dq=lambda e: O.dequant_int4_group(c[0][e], c[1][e]),
                                       w2_dq=lambda e: O.dequant_int4_group(c[2][e], c[3][e]))
    else:
        q1, q2 = _weights(H, E, I)
        s1 = s2 = None
        code = _lib.QUANT_NONE
        ref = O.fused_experts_rounding(x.cpu(), q1.cpu(), q2.cpu(), rw, rids)
    out, tw, ti = ops.moe_block(x, wg, q1, q2, k, True, 0, code, s1, s2)
    assert torch.equal(ti.cpu(), rids)
    torch.testing.assert_close(tw.cpu(), rw, rtol=2e-6, atol=1e-9)
    assert_moe_close(out, ref, what=f"moe_block M={M} {quant}")


def test_sparse_moe_block_uses_one_call():
    """SparseMoeBlock.routed with the default bf16 router runs moe_block
    (and equals the router + fused_experts composition bit for bit)."""
    from mstar_amd import ops
    from mstar_amd.fused_moe import fused_experts
    from mstar_amd.moe import SparseMoeBlock
    torch.manual_seed(3)
    H, E, I, k = 2048, 128, 768, 8
    blk = SparseMoeBlock(H, E, k, I).to(DEV, torch.bfloat16)
    with torch.no_grad():
        blk.experts.gate_up_proj.normal_(std=0.02)
        blk.experts.down_proj.normal_(std=0.02)
        blk.gate.weight.normal_(std=0.05)
    blk.quantize("fp8_w8a8")
    x = torch.randn(32, H, device=DEV, dtype=torch.bfloat16)
    calls = []
    real = ops.moe_block

    def spy(*a, **kw):
        calls.append(1)
        return real(*a, **kw)

    ops.moe_block = spy
    try:
        out = blk(x)
    finally:
        ops.moe_block = real
    assert calls == [1]
    w, ids = ops.router(x, blk.gate.weight, k, True)
    ex = blk.experts
    ref = fused_experts(x, ex.gate_up_proj, ex.down_proj, w, ids, quant="fp8_w8a8",
                        w1_scale=ex.w1_scale, w2_scale=ex.w2_scale)
    assert torch.equal(out, ref)


def test_fp16_block_and_router():
    """A block in fp16 (the reference's blocks run in the model dtype): the
    gate projection in fp16, routing from fp16 logits, fp16 experts."""
    from mstar_amd.moe import SparseMoeBlock, TopKRouter
    torch.manual_seed(4)
    H, E, I, k = 1024, 128, 384, 8
    blk = SparseMoeBlock(H, E, k, I).to(DEV, torch.float16)
    with torch.no_grad():
        blk.experts.gate_up_proj.normal_(std=0.02)
        blk.experts.down_proj.normal_(std=0.02)
        blk.gate.weight.normal_(std=0.05)
    x = torch.randn(40, H, device=DEV, dtype=torch.float16)
    out = blk(x)
    assert out.dtype == torch.float16
    logits = torch.nn.functional.linear(x, blk.gate.weight)
    rw, rids = O.router_topk_softmax(logits.cpu(), k, True)
    ref = O.fused_experts_rounding(x.cpu(), blk.experts.gate_up_proj.detach().cpu(),
                                   blk.experts.down_proj.detach().cpu(), rw, rids)
    assert_moe_close(out, ref, what="fp16 SparseMoeBlock")
    r = TopKRouter(H, E, k).to(DEV, torch.float16)
    with torch.no_grad():
        r.weight.copy_(blk.gate.weight)
    w, ids, _ = r(x)
    assert torch.equal(ids.cpu(), rids)
    torch.testing.assert_close(w.cpu(), rw, rtol=2e-6, atol=1e-9)


def test_layer_from_saved_fp8_experts(tmp_path):
    """Per-expert, per-rank loaders (tp 2, rank 1) -> safetensors -> load ->
    fused_experts on the GPU, against the oracle on the loaded tensors and
    against quantising the rank's bf16 slice directly."""
    from mstar_amd import quant as Q
    from mstar_amd import weights as W
    from mstar_amd.fused_moe import fused_experts
    H, E, I_full, k, tp, rank = 1024, 16, 768, 4, 2, 1
    g = torch.Generator().manual_seed(5)
    gate = torch.randn(E, I_full, H, generator=g) * 0.02
    up = torch.randn(E, I_full, H, generator=g) * 0.02
    down = torch.randn(E, H, I_full, generator=g) * 0.02
    w1_q, w1_s, w2_q, w2_s = W.empty_fp8_experts(E, H, I_full, tp)
    for e in range(E):
        W.fp8_gate_up_weight_loader(rank, tp, I_full, w1_q, w1_s, gate[e].to(torch.bfloat16), f"gate:{e}")
        W.fp8_gate_up_weight_loader(rank, tp, I_full, w1_q, w1_s, up[e].to(torch.bfloat16), f"up:{e}")
        W.fp8_down_proj_weight_loader(rank, tp, I_full, w2_q, w2_s, down[e].to(torch.bfloat16), f"down:{e}")
    path = str(tmp_path / "experts.safetensors")
    W.save_fp8_experts(path, w1_q, w1_s, w2_q, w2_s)
    q1, s1, q2, s2 = W.load_fp8_experts(path, device=DEV)
    Ip = I_full // tp
    sl = slice(rank * Ip, (rank + 1) * Ip)
    stack1 = torch.cat([gate[:, sl], up[:, sl]], dim=1).to(torch.bfloat16)
    d1, e1 = Q.quantize_fp8_block(stack1)
    assert torch.equal(q1.cpu().view(torch.uint8), d1.view(torch.uint8)) and torch.equal(s1.cpu(), e1)
    M = 300
    x = _hidden(M, H, seed=6)
    tw, ti = _routing(M, E, k, seed=6)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, tw, ti), what="saved fp8 experts")


def _int4_plain(w: torch.Tensor):
    """Symmetric int4 per 128-group with plain bf16 scales amax / 7 (any
    mantissa), packed as the W4A16 kernels read it (q + 8 in bits 4 (k % 8)
    of word k / 8).  Returns (packed, scales, exact dequant fp32)."""
    *lead, N, K = w.shape
    wf = w.float().view(*lead, N, K // 128, 128)
    s = (wf.abs().amax(dim=-1).clamp_min(1e-10) / 7.0).to(torch.bfloat16)
    q = torch.round(wf / s.float()[..., None]).clamp(-8, 7).to(torch.int32)
    deq = (q.float() * s.float()[..., None]).view(*lead, N, K)  # exact: 4 x 8 bits in fp32
    u = (q.view(*lead, N, K) + 8).view(*lead, N, K // 8, 8)
    packed = torch.zeros(*lead, N, K // 8, dtype=torch.int32, device=w.device)
    for i in range(8):
        packed |= u[..., i] << (4 * i)
    return packed.contiguous(), s.contiguous(), deq


@pytest.mark.parametrize("M", [1, 32, 300, 1024])
def test_w4a16_plain_scales(M):
    """Every W4A16 regime (decode streaming, 64-token tiles, Zipf-skewed
    prefill) on unrestricted scales: against the oracle's rounding points on
    the exact dequantised weights, and within bf16 noise of float64."""
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 8
    w1, w2 = _weights(H, E, I, seed=8)
    p1, t1, d1 = _int4_plain(w1.cpu())
    p2, t2, d2 = _int4_plain(w2.cpu())
    assert (t1.view(torch.int16) & 0x3).any()  # scales using all 8 significant bits of bf16
    x = _hidden(M, H, seed=M + 8)
    tw, ti = _routing(M, E, k, seed=M + 8, bias=M >= 300)
    out = fused_experts(x.to(DEV), p1.to(DEV), p2.to(DEV), tw.to(DEV), ti.to(DEV), quant="w4a16",
                        w1_scale=t1.to(DEV), w2_scale=t2.to(DEV))
    ref = O.fused_experts_rounding(x, None, None, tw, ti, w1_dq=lambda e: d1[e], w2_dq=lambda e: d2[e])
    assert_moe_close(out, ref, what=f"w4a16 plain scales M={M}")
    n = min(M, 8)
    f64 = O.textbook_moe_f64(x[:n], d1, d2, tw[:n], ti[:n])
    assert_moe_close(out[:n], f64, max_rel=3e-2, mean_of_rms=1e-2, what=f"w4a16 plain vs f64 M={M}")


def test_public_ops_reject_bad_arguments():
    from mstar_amd import _lib, ops
    H, E, I, k, M = 256, 8, 256, 2, 4
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = torch.randn(M, H, device=DEV).to(torch.bfloat16)
    tw = torch.full((M, k), 0.5, device=DEV)
    ti = torch.randint(0, E, (M, k), device=DEV)
    F8 = _lib.QUANT_FP8_W8A8

    def run(**over):
        a = dict(hidden=x, w1=q1, w2=q2, topk_weights=tw, topk_ids=ti, activation=0,
                 reduce_results=True, quant=F8, w1_scale=s1, w2_scale=s2)
        a.update(over)
        return ops.fused_experts_op(**a)

    assert run().shape == (M, H)
    bad = [
        dict(w1_scale=s1.to(torch.bfloat16)),                          # dtype
        dict(w1_scale=s1[:, :1].contiguous()),                         # per-channel-like shape
        dict(w2_scale=s2.transpose(1, 2)),                             # transposed
        dict(w2_scale=torch.empty_like(s2).transpose(1, 2).contiguous().transpose(1, 2)),  # strided
        dict(w1_scale=None),
        dict(topk_ids=ti[:M - 1], topk_weights=tw[:M - 1]),            # rows != tokens
        dict(topk_ids=ti[:, :1]),                                      # ids / weights mismatch
        dict(topk_ids=ti.to(torch.int16)),
        dict(w1=q1[0]),                                                # not [E, ., .]
        dict(w2=q2[:, :, :128]),                                       # inter mismatch
    ]
    for b in bad:
        with pytest.raises((ValueError, TypeError)):
            run(**b)
    with pytest.raises(ValueError):
        ops.moe_sum_reduce(torch.zeros(M, k, H, device=DEV, dtype=torch.bfloat16),
                           torch.empty(M, H, device=DEV, dtype=torch.float16), 1.0)
    with pytest.raises(ValueError):
        ops.moe_layer(x, torch.zeros(M + 1, E, device=DEV), q1, q2, k, True, 0, F8, s1, s2)
    with pytest.raises(ValueError):
        ops.moe_block(x, torch.zeros(E, H + 32, device=DEV, dtype=torch.bfloat16), q1, q2, k, True,
                      0, F8, s1, s2)
