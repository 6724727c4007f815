"""GPU parity of the fused MoE path against the oracle.

Tolerance (floating point): max|out-ref| <= 2e-2 * max|ref| and
mean|out-ref| <= 1e-3 * rms(ref) against the rounding-point oracle
(tests/_util.py); plus the reference test's own bar, assert_close(atol=rtol=
2e-2) against the naive per-expert path
(test/modular/test_qwen3_omni_fused_moe.py:102).
"""
from __future__ import annotations

import functools
import os

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@functools.lru_cache(maxsize=4)
def _weights(H, E, I, seed=0, dtype=torch.bfloat16):
    """Seeded expert weights, generated on the GPU (fast) and kept on both sides."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    w1 = (torch.randn(E, 2 * I, H, generator=g, device=DEV) * 0.02).to(dtype)
    w2 = (torch.randn(E, H, I, generator=g, device=DEV) * 0.02).to(dtype)
    return w1, w2


def _routing(M, E, k, seed=0, bias=False, renorm=True):
    g = torch.Generator().manual_seed(seed + 17)
    logits = torch.randn(M, E, generator=g)
    if bias:
        logits = logits + O.zipf_bias(E)
    return O.router_topk_softmax(logits, k, renorm)


def _hidden(M, H, seed=0, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed + 99)
    return torch.randn(M, H, generator=g).to(dtype)


# ------------------------------------------------------------------ bf16
@pytest.mark.parametrize("num_tokens", [1, 4, 16, 64])
@pytest.mark.parametrize("hidden,inter,num_experts,top_k", [(2048, 768, 128, 8), (1024, 384, 128, 8)])
def test_fused_experts_bf16_reference_shapes(num_tokens, hidden, inter, num_experts, top_k):
    from mstar_amd.fused_moe import fused_experts
    w1, w2 = _weights(hidden, num_experts, inter)
    x = _hidden(num_tokens, hidden)
    tw, ti = _routing(num_tokens, num_experts, top_k)
    out = fused_experts(x.to(DEV), w1, w2, tw.to(DEV), ti.to(DEV))
    torch.cuda.synchronize()
    assert out.shape == x.shape and out.dtype == torch.bfloat16
    w1c, w2c = w1.cpu(), w2.cpu()
    ref = O.fused_experts_rounding(x, w1c, w2c, tw, ti)
    assert_moe_close(out, ref, what="fused bf16 vs oracle")
    naive = O.naive_dispatch(x, w1c, w2c, num_experts, ti, tw.to(torch.bfloat16))
    torch.testing.assert_close(out.cpu(), naive, atol=2e-2, rtol=2e-2)


def test_fused_experts_tiny_config_vs_golden():
    from mstar_amd.fused_moe import fused_experts
    x, w1, w2, logits = O.make_moe_inputs(64, 256, 8, 2, 512, seed=0)
    g = np.load(os.path.join(GOLDEN, "moe_tiny_bf16.npz"), allow_pickle=False)
    w, ids = O.router_topk_softmax(logits, 2, True)
    assert np.array_equal(ids.numpy(), g["topk_ids"])
    out = fused_experts(x.to(DEV), w1.to(DEV), w2.to(DEV), w.to(DEV), ids.to(DEV))
    ref = torch.from_numpy(g["out_bits"]).view(torch.bfloat16)
    naive = torch.from_numpy(g["naive_bits"]).view(torch.bfloat16)
    assert_moe_close(out, ref, what="tiny vs golden")
    torch.testing.assert_close(out.cpu(), naive, atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("M,E,k,H,I", [(300, 16, 4, 256, 256), (1024, 8, 2, 256, 384)])
def test_fused_experts_bf16_large_blocks(M, E, k, H, I):
    from mstar_amd.fused_moe import fused_experts
    w1, w2 = _weights(H, E, I, seed=3)
    x = _hidden(M, H, seed=3)
    tw, ti = _routing(M, E, k, seed=3)
    out = fused_experts(x.to(DEV), w1, w2, tw.to(DEV), ti.to(DEV))
    ref = O.fused_experts_rounding(x, w1.cpu(), w2.cpu(), tw, ti)
    assert_moe_close(out, ref, what=f"bf16 M={M}")


def test_fused_experts_fp16_gelu_unreduced():
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k, M = 256, 8, 256, 2, 40
    w1, w2 = _weights(H, E, I, seed=5, dtype=torch.float16)
    x = _hidden(M, H, seed=5, dtype=torch.float16)
    tw, ti = _routing(M, E, k, seed=5)
    out = fused_experts(x.to(DEV), w1, w2, tw.to(DEV).half(), ti.to(DEV).int(), activation="gelu",
                        reduce_results=False)
    assert out.shape == (M, k, H) and out.dtype == torch.float16
    ref = O.fused_experts_rounding(x, w1.cpu(), w2.cpu(), tw.half(), ti, activation="gelu",
                                   reduce_results=False)
    assert_moe_close(out, ref, what="fp16 gelu unreduced")


@pytest.mark.parametrize("quant,M", [("fp8_w8a8", 32), ("fp8_w8a8", 300), ("fp8_w8a8", 4096),
                                     ("w4a16", 32), ("w4a16", 300)])
@pytest.mark.parametrize("reduce", [True, False])
def test_fused_experts_quantised_gelu(quant, M, reduce):
    """GeLU (tanh) through every quantised path -- decode streaming (M=32),
    mid-size tiles (M=300: FP8 128-row tiles, int4 64x256 tiles) and the
    256-row FP8 kernel (M=4096) -- with and without the top-k sum."""
    from mstar_amd import quant as Q
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 8
    x = _hidden(M, H, seed=M + 7)
    tw, ti = _routing(M, E, k, seed=M + 7)
    if quant == "fp8_w8a8":
        q1, s1, q2, s2 = _fp8_weights(H, E, I)
        c1, c2, c3, c4 = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
        d1 = lambda e: O.dequant_fp8_block(c1[e], c2[e])
        d2 = lambda e: O.dequant_fp8_block(c3[e], c4[e])
        kw = dict(block_shape=(128, 128))
        aq = True
    else:
        w1, w2 = _weights(H, E, I)
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        c1, c2, c3, c4 = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
        d1 = lambda e: O.dequant_int4_group(c1[e], c2[e])
        d2 = lambda e: O.dequant_int4_group(c3[e], c4[e])
        kw = {}
        aq = False
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), activation="gelu",
                        reduce_results=reduce, quant=quant, w1_scale=s1, w2_scale=s2, **kw)
    ref = O.fused_experts_rounding(x, None, None, tw, ti, activation="gelu", reduce_results=reduce,
                                   w1_dq=d1, w2_dq=d2, act_quant=aq)
    assert_moe_close(out, ref, what=f"{quant} gelu M={M} reduce={reduce}")


def test_reference_api_composition():
    """The reference runner's own sequence (runner.py:99-159) through the
    drop-in kernel entry points: align -> GEMM1 -> act_and_mul -> GEMM2 ->
    sum-reduce, at the reference's block sizes."""
    from mstar_amd.fused_moe import (act_and_mul_triton, get_default_config,
                                     invoke_fused_moe_kernel, moe_align_block_size,
                                     moe_sum_reduce_triton)
    for M in (16, 300):
        H, E, I, k = 256, 32, 256, 4
        w1, w2 = _weights(H, E, I, seed=6)
        x = _hidden(M, H, seed=6).to(DEV)
        tw, ti = _routing(M, E, k, seed=6)
        tw_d, ti_d = tw.to(DEV), ti.to(DEV).int()
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
        assert_moe_close(out, ref, what=f"reference composition M={M}")


# ------------------------------------------------------------------- FP8
@functools.lru_cache(maxsize=2)
def _fp8_weights(H, E, I, seed=0):
    from mstar_amd import quant
    w1, w2 = _weights(H, E, I, seed=seed)
    q1, s1 = quant.quantize_fp8_block(w1)
    q2, s2 = quant.quantize_fp8_block(w2)
    return q1, s1, q2, s2


def _fp8_ref(x, q1, s1, q2, s2, tw, ti):
    q1c, s1c, q2c, s2c = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
    d1 = lambda e: O.dequant_fp8_block(q1c[e], s1c[e])
    d2 = lambda e: O.dequant_fp8_block(q2c[e], s2c[e])
    return O.fused_experts_rounding(x, None, None, tw, ti, w1_dq=d1, w2_dq=d2, act_quant=True)


@pytest.mark.parametrize("M,bias", [(32, False), (1, False), (64, True), (512, True), (2048, True),
                                    (2048, False)])
def test_fused_experts_fp8_thinker(M, bias):
    """Config 2 (decode, M=32; weight-streaming path for M <= 64) and config 3
    (prefill with the Zipf bias; tiled path) at Qwen3-30B-A3B thinker shapes."""
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 8
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = _hidden(M, H, seed=M)
    tw, ti = _routing(M, E, k, seed=M, bias=bias)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2, block_shape=(128, 128))
    ref = _fp8_ref(x, q1, s1, q2, s2, tw, ti)
    assert_moe_close(out, ref, what=f"fp8 M={M}")


def test_moe_layer_prefill_8192_zipf_rows():
    """Config 3's headline point: 8192 tokens, Zipf-biased routing (expert 0
    takes thousands of slots), the whole layer from logits.  Each token's
    output depends on its own row only (its activation quantisation is per
    token and group), so the oracle scores 320 fixed rows: the first 128,
    128 routed to expert 0 and 64 spread over the batch."""
    from mstar_amd import _lib, ops
    M, H, E, I, k = 8192, 2048, 128, 768, 8
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = _hidden(M, H, seed=8192)
    g = torch.Generator().manual_seed(8193)
    logits = torch.randn(M, E, generator=g) + O.zipf_bias(E)
    rw, rids = O.router_topk_softmax(logits, k, True)
    out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8,
                                s1, s2)
    assert torch.equal(ti.cpu(), rids)
    to_e0 = torch.nonzero((rids == 0).any(dim=1)).flatten()
    assert to_e0.numel() > 1000  # the skew the bench times
    rows = torch.cat([torch.arange(128), to_e0[torch.randperm(to_e0.numel(), generator=g)[:128]],
                      torch.randint(0, M, (64,), generator=g)]).unique()
    ref = _fp8_ref(x[rows], q1, s1, q2, s2, rw[rows], rids[rows])
    assert_moe_close(out.cpu()[rows], ref, what="moe_layer fp8 M=8192 zipf rows")


@pytest.mark.parametrize("M", [16384, 65536])
def test_moe_layer_large_batches(M):
    """Batches past the bench's prefill point (131072 and 524288 slots): the
    grid-wide routing over 512 / 2048 workgroups, 32-bit position offsets
    and the 256-row GEMMs at eight times the M=8192 tile count.  Routing is
    checked whole; the oracle scores the first and last 64 rows and 128 in
    between."""
    from mstar_amd import _lib, ops
    H, E, I, k = 2048, 128, 768, 8
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    g = torch.Generator().manual_seed(M)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g) + O.zipf_bias(E)
    rw, rids = O.router_topk_softmax(logits, k, True)
    print(f"moe_layer large batch M={M}", flush=True)
    out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0, _lib.QUANT_FP8_W8A8,
                                s1, s2)
    assert torch.equal(ti.cpu(), rids)
    rows = torch.cat([torch.arange(64), torch.randint(0, M, (128,), generator=g),
                      torch.arange(M - 64, M)]).unique()
    ref = _fp8_ref(x[rows], q1, s1, q2, s2, rw[rows], rids[rows])
    assert_moe_close(out.cpu()[rows], ref, what=f"moe_layer fp8 M={M} zipf rows")


@pytest.mark.parametrize("reduce", [True, False])
def test_fused_experts_fp8_position_rows(reduce):
    """4096 tokens x top-8 over 128 experts: the 256-row FP8 kernel stores the
    intermediates by sorted position; with reduce_results=False the down GEMM
    writes per slot ([tokens, top_k, hidden]) from position-indexed inputs."""
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k, M = 2048, 128, 768, 8, 4096
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    x = _hidden(M, H, seed=41)
    tw, ti = _routing(M, E, k, seed=41, bias=True)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2, block_shape=(128, 128), reduce_results=reduce)
    q1c, s1c, q2c, s2c = q1.cpu(), s1.cpu(), q2.cpu(), s2.cpu()
    ref = O.fused_experts_rounding(x, None, None, tw, ti, reduce_results=reduce,
                                   w1_dq=lambda e: O.dequant_fp8_block(q1c[e], s1c[e]),
                                   w2_dq=lambda e: O.dequant_fp8_block(q2c[e], s2c[e]), act_quant=True)
    assert_moe_close(out, ref, what=f"fp8 position rows reduce={reduce}")


def test_fused_experts_fp8_bm128_path():
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k, M = 256, 8, 256, 2, 1024
    q1, s1, q2, s2 = _fp8_weights(H, E, I, seed=7)
    x = _hidden(M, H, seed=7)
    tw, ti = _routing(M, E, k, seed=7)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, tw, ti), what="fp8 bm128")


@pytest.mark.parametrize("H,I,E,k,M", [(256, 256, 4, 2, 200), (512, 256, 8, 1, 100), (256, 512, 2, 2, 130),
                                       (2048, 768, 128, 8, 65)])
def test_fused_experts_w4a16_tile_shapes(H, I, E, k, M):
    """The int4 tile GEMM at its edges: one K-step per tile (the next tile's
    first step issued in the same iteration), a single n-tile, top-1, fewer
    tiles than CUs, and the smallest token count above the streaming path."""
    from mstar_amd import quant
    from mstar_amd.fused_moe import fused_experts
    w1, w2 = _weights(H, E, I, seed=H + I + E)
    p1, t1 = quant.quantize_int4_group(w1)
    p2, t2 = quant.quantize_int4_group(w2)
    x = _hidden(M, H, seed=M + E)
    tw, ti = _routing(M, E, k, seed=M + k)
    out = fused_experts(x.to(DEV), p1, p2, tw.to(DEV), ti.to(DEV), quant="w4a16",
                        w1_scale=t1, w2_scale=t2)
    p1c, t1c, p2c, t2c = p1.cpu(), t1.cpu(), p2.cpu(), t2.cpu()
    ref = O.fused_experts_rounding(x, None, None, tw, ti,
                                   w1_dq=lambda e: O.dequant_int4_group(p1c[e], t1c[e]),
                                   w2_dq=lambda e: O.dequant_int4_group(p2c[e], t2c[e]))
    assert_moe_close(out, ref, what=f"w4a16 tile H={H} I={I} E={E} k={k} M={M}")


def test_weight_quant_matches_oracle():
    from mstar_amd import quant
    w1, _ = _weights(256, 4, 128, seed=8)
    q, s = quant.quantize_fp8_block(w1)
    rq, rs = O.quant_fp8_block(w1.cpu())
    assert torch.equal(q.cpu().view(torch.uint8), rq.view(torch.uint8))
    assert torch.equal(s.cpu(), rs)
    p, t = quant.quantize_int4_group(w1)
    rp, rt = O.quant_int4_group(w1.cpu())
    assert torch.equal(p.cpu(), rp) and torch.equal(t.cpu(), rt)


# ----------------------------------------------------------------- W4A16
@pytest.mark.parametrize("M", [32, 1, 256, 1024])
def test_fused_experts_w4a16_thinker(M):
    """Config 5 at the decode shapes (M=32 streaming; M=256/1024 tiled)."""
    from mstar_amd import quant
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 8
    w1, w2 = _weights(H, E, I)
    p1, t1 = quant.quantize_int4_group(w1)
    p2, t2 = quant.quantize_int4_group(w2)
    x = _hidden(M, H, seed=M + 1)
    tw, ti = _routing(M, E, k, seed=M + 1)
    out = fused_experts(x.to(DEV), p1, p2, tw.to(DEV), ti.to(DEV), quant="w4a16",
                        w1_scale=t1, w2_scale=t2)
    p1c, t1c, p2c, t2c = p1.cpu(), t1.cpu(), p2.cpu(), t2.cpu()
    ref = O.fused_experts_rounding(x, None, None, tw, ti,
                                   w1_dq=lambda e: O.dequant_int4_group(p1c[e], t1c[e]),
                                   w2_dq=lambda e: O.dequant_int4_group(p2c[e], t2c[e]))
    assert_moe_close(out, ref, what=f"w4a16 M={M}")


# ----------------------------------------------------------------- blocks
def test_sparse_moe_block_and_shared_expert():
    from mstar_amd.moe import SparseMoeBlock, SparseMoeBlockWithSharedExpert
    torch.manual_seed(0)
    H, E, I, k = 1024, 128, 384, 8
    blk = SparseMoeBlock(H, E, k, I, norm_topk_prob=True).to(DEV, torch.bfloat16)
    with torch.no_grad():
        blk.experts.gate_up_proj.normal_(std=0.02)
        blk.experts.down_proj.normal_(std=0.02)
        blk.gate.weight.normal_(std=0.02)
    x = torch.randn(16, H, device=DEV, dtype=torch.bfloat16)
    out = blk(x)
    # bf16 logits: exact ties are common; the kernel and the oracle both
    # order them lower-index first, so the ids must agree exactly.
    logits = torch.nn.functional.linear(x, blk.gate.weight)
    gw, gi, _ = blk.gate(x)
    tw, ti = O.router_topk_softmax(logits.cpu(), k, True)
    assert torch.equal(gi.cpu(), ti)
    torch.testing.assert_close(gw.cpu(), tw, rtol=2e-6, atol=1e-9)
    ref = O.fused_experts_rounding(x.cpu(), blk.experts.gate_up_proj.detach().cpu(),
                                   blk.experts.down_proj.detach().cpu(), tw, ti)
    assert_moe_close(out, ref, what="SparseMoeBlock")
    out2, state = blk(x, return_router_states=True)
    assert state is None and torch.equal(out, out2)

    shared = torch.nn.Linear(H, H, bias=False).to(DEV, torch.bfloat16)
    sb = SparseMoeBlockWithSharedExpert(H, E, k, I, shared_expert=shared).to(DEV, torch.bfloat16)
    sb.load_state_dict(blk.state_dict(), strict=False)
    with torch.no_grad():
        sb.shared_expert_gate.weight.normal_(std=0.02)
    out3 = sb(x)
    tw2, ti2 = O.router_topk_softmax(logits.cpu(), k, False)
    routed = O.fused_experts_rounding(x.cpu(), blk.experts.gate_up_proj.detach().cpu(),
                                      blk.experts.down_proj.detach().cpu(), tw2, ti2)
    ref3 = routed + torch.sigmoid(sb.shared_expert_gate(x)).cpu() * shared(x).cpu()
    assert_moe_close(out3, ref3, what="shared-expert block")


def test_block_quantize_fp8():
    from mstar_amd.moe import SparseMoeBlock
    H, E, I, k = 1024, 128, 384, 8
    blk = SparseMoeBlock(H, E, k, I).to(DEV, torch.bfloat16)
    with torch.no_grad():
        blk.experts.gate_up_proj.normal_(std=0.02)
        blk.experts.down_proj.normal_(std=0.02)
        blk.gate.weight.normal_(std=0.02)
    x = torch.randn(8, H, device=DEV, dtype=torch.bfloat16)
    ref = blk(x)
    blk.quantize("fp8_w8a8")
    out = blk(x)
    # FP8 weights and activations: within a few percent of the bf16 block.
    err = (out.float() - ref.float()).abs().max() / ref.float().abs().max()
    assert float(err) < 0.1


# ----------------------------------------------------------- graph capture
def test_layer_under_hip_graph_replays():
    """Route + fused FP8 layer captured in a HIP graph: every replay (with
    eager work and syncs in between) equals the eager result bit for bit."""
    from mstar_amd import ops
    from mstar_amd.fused_moe import fused_experts
    H, E, I, k = 2048, 128, 768, 8
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    for M in (32, 300):
        x = _hidden(M, H, seed=11).to(DEV)
        logits = torch.randn(M, E, device=DEV)

        def fn():
            w, ids = ops.topk_softmax(logits, k, True)
            return fused_experts(x, q1, q2, w, ids, quant="fp8_w8a8", w1_scale=s1, w2_scale=s2)

        eager = fn()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = fn()
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            _ = fn()  # eager work between replays
            torch.cuda.synchronize()


@pytest.mark.parametrize("M,bias,quant", [(32, False, "fp8_w8a8"), (8, False, "fp8_w8a8"),
                                          (512, True, "fp8_w8a8"), (1024, True, "fp8_w8a8"),
                                          (4096, True, "fp8_w8a8"), (16, False, None),
                                          (32, False, "w4a16"), (1024, True, "w4a16")])
def test_moe_layer_from_logits(M, bias, quant):
    """Routing from logits + experts in one library call (mstar_moe_layer).
    Above 512 slots the multi-workgroup routing also quantises the hidden
    rows; from M=384 (24 slots per expert) the FP8 tile kernel runs, on 128-row
    tiles below 128 slots per expert (M=512, 1024) and 256-row tiles above
    (M=4096); W4A16 at M=1024 (Zipf routing: experts spanning many 64-token
    blocks) runs the int4 tile GEMM."""
    from mstar_amd import _lib, ops, quant as Q
    H, E, I, k = 2048, 128, 768, 8
    x = _hidden(M, H, seed=M + 21)
    g = torch.Generator().manual_seed(M + 22)
    logits = torch.randn(M, E, generator=g)
    if bias:
        logits = logits + O.zipf_bias(E)
    rw, rids = O.router_topk_softmax(logits, k, True)
    w1, w2 = _weights(H, E, I)
    if quant == "fp8_w8a8":
        q1, s1, q2, s2 = _fp8_weights(H, E, I)
        out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, True, 0,
                                    _lib.QUANT_FP8_W8A8, s1, s2)
        ref = _fp8_ref(x, q1, s1, q2, s2, rw, rids)
    elif quant == "w4a16":
        p1, t1 = Q.quantize_int4_group(w1)
        p2, t2 = Q.quantize_int4_group(w2)
        out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), p1, p2, k, True, 0,
                                    _lib.QUANT_W4A16, t1, t2)
        p1c, t1c, p2c, t2c = p1.cpu(), t1.cpu(), p2.cpu(), t2.cpu()
        ref = O.fused_experts_rounding(x, None, None, rw, rids,
                                       w1_dq=lambda e: O.dequant_int4_group(p1c[e], t1c[e]),
                                       w2_dq=lambda e: O.dequant_int4_group(p2c[e], t2c[e]))
    else:
        out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), w1, w2, k, True, 0,
                                    _lib.QUANT_NONE, None, None)
        ref = O.fused_experts_rounding(x, w1.cpu(), w2.cpu(), rw, rids)
    assert torch.equal(ti.cpu(), rids)
    torch.testing.assert_close(tw.cpu(), rw, rtol=2e-6, atol=1e-9)
    assert_moe_close(out, ref, what=f"moe_layer M={M} {quant}")


@pytest.mark.parametrize("M,renorm,E,k", [(24, False, 128, 8), (32, True, 128, 8), (5, True, 128, 8),
                                          (16, True, 64, 6), (8, False, 100, 8)])
def test_moe_layer_decode_bf16_logits(M, renorm, E, k):
    """Decode layers (routing launch + router-ids GEMMs): bf16 logits (with
    exact ties), both renormalisation settings and expert counts that are not
    a multiple of 16 give the oracle's routing and output."""
    from mstar_amd import _lib, ops
    H, I = 2048, 768
    x = _hidden(M, H, seed=M + 31)
    g = torch.Generator().manual_seed(M + 32)
    logits = (torch.randn(M, E, generator=g) * 0.5).to(torch.bfloat16)
    rw, rids = O.router_topk_softmax(logits.float(), k, renorm)
    q1, s1, q2, s2 = _fp8_weights(H, E, I)
    out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, k, renorm, 0,
                                _lib.QUANT_FP8_W8A8, s1, s2)
    assert torch.equal(ti.cpu(), rids)
    torch.testing.assert_close(tw.cpu(), rw, rtol=2e-6, atol=1e-9)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, rw, rids), what=f"decode layer bf16 logits M={M} E={E}")


@pytest.mark.parametrize("M,E,k,H,I,bias", [(1024, 16, 4, 512, 256, False), (2048, 32, 8, 1024, 384, True)])
def test_fused_experts_fp8_big_tile_path(M, E, k, H, I, bias):
    """>= 24 slots per expert on average selects the 256 x 256 FP8 tile kernel."""
    from mstar_amd.fused_moe import fused_experts
    q1, s1, q2, s2 = _fp8_weights(H, E, I, seed=9)
    x = _hidden(M, H, seed=9)
    tw, ti = _routing(M, E, k, seed=9, bias=bias)
    out = fused_experts(x.to(DEV), q1, q2, tw.to(DEV), ti.to(DEV), quant="fp8_w8a8",
                        w1_scale=s1, w2_scale=s2)
    assert_moe_close(out, _fp8_ref(x, q1, s1, q2, s2, tw, ti), what=f"fp8 big tile M={M}")


@pytest.mark.parametrize("quant", ["fp8_w8a8", "w4a16"])
def test_one_launch_layer_under_hip_graph_replays(quant):
    """mstar_moe_layer at decode size (routing launch, then the experts in one
    launch whose per-expert counters the routing launch clears) captured three
    layers to a graph: every replay equals the eager result bit for bit, with
    eager layers in between, and no wait of the layer kernel gave up."""
    import ctypes
    from mstar_amd import _lib, ops, quant as Q
    H, E, I, k, M = 2048, 128, 768, 8, 32
    if quant == "fp8_w8a8":
        q1, s1, q2, s2 = _fp8_weights(H, E, I)
        qc = _lib.QUANT_FP8_W8A8
    else:
        g = torch.Generator().manual_seed(5)
        w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(DEV)
        w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(DEV)
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        qc = _lib.QUANT_W4A16
    xs = [_hidden(M, H, seed=40 + i).to(DEV) for i in range(3)]
    ls = [torch.randn(M, E, device=DEV) for _ in range(3)]

    def fn():
        return [ops.moe_layer(x, l, q1, q2, k, True, 0, qc, s1, s2)[0] for x, l in zip(xs, ls)]

    n0 = ctypes.c_int(-1)
    _lib.check(_lib.load().mstar_moe_layer_wait_failures(ctypes.byref(n0)), "moe_layer_wait_failures")
    eager = [o.clone() for o in fn()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = fn()
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)
        _ = fn()
        torch.cuda.synchronize()
    n = ctypes.c_int(-1)
    _lib.check(_lib.load().mstar_moe_layer_wait_failures(ctypes.byref(n)), "moe_layer_wait_failures")
    assert n.value == n0.value
