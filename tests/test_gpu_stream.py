"""Decode entry points driven directly by the router ids (no alignment step):
mstar_moe_topk_softmax_quant and mstar_moe_stream_gemm, composed the way the
reference runner composes its stages (mstar/utils/fused_moe/runner.py:99-159)
and checked against the CPU oracle."""
from __future__ import annotations

import functools

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close

pytestmark = pytest.mark.gpu
DEV = "cuda"
H, E, I, K_TOP = 2048, 128, 768, 8


@functools.lru_cache(maxsize=1)
def _weights():
    from mstar_amd import quant
    g = torch.Generator().manual_seed(11)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(DEV)
    q1, s1 = quant.quantize_fp8_block(w1)
    q2, s2 = quant.quantize_fp8_block(w2)
    return q1, s1, q2, s2


def _inputs(M, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g)
    return x, logits


def _ref(x, tw, ti):
    q1, s1, q2, s2 = (t.cpu() for t in _weights())
    d1 = lambda e: O.dequant_fp8_block(q1[e], s1[e])
    d2 = lambda e: O.dequant_fp8_block(q2[e], s2[e])
    return O.fused_experts_rounding(x, None, None, tw, ti, w1_dq=d1, w2_dq=d2, act_quant=True)


def _route_quant(x, logits):
    from mstar_amd import _lib
    lib = _lib.load()
    M = x.shape[0]
    tw = torch.empty(M, K_TOP, dtype=torch.float32, device=DEV)
    ti = torch.empty(M, K_TOP, dtype=torch.int32, device=DEV)
    hq = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    hs = torch.empty(M, H // 128, dtype=torch.float32, device=DEV)
    xd, ld = x.to(DEV), logits.to(DEV)
    _lib.check(lib.mstar_moe_topk_softmax_quant(
        ld.data_ptr(), _lib.DT_F32, M, E, K_TOP, 1, tw.data_ptr(), ti.data_ptr(), None,
        xd.data_ptr(), H, hq.data_ptr(), hs.data_ptr(), _lib.stream_of(xd)), "topk_softmax_quant")
    return tw, ti, hq, hs


def _stream_gemm(A, a_dt, a_scale, B, b_scale, C, tw, ti, slots, N, Kd, top_k, mul, act):
    from mstar_amd import _lib
    lib = _lib.load()
    _lib.check(lib.mstar_moe_stream_gemm(
        A.data_ptr(), a_dt, _lib.ptr(a_scale), B.data_ptr(), b_scale.data_ptr(), C.data_ptr(),
        tw.data_ptr(), _lib.DT_F32, ti.data_ptr(), _lib.dtype_code(ti.dtype), slots, E, N, Kd,
        top_k, mul, act, _lib.stream_of(A)), "moe_stream_gemm")


def test_topk_softmax_quant_bit_exact():
    """Routing equals mstar_moe_topk_softmax; the widened codes and scales
    equal the per-token-group quantisation of the oracle bit for bit."""
    from mstar_amd import ops
    x, logits = _inputs(32, seed=1)
    tw, ti, hq, hs = _route_quant(x, logits)
    tw2, ti2 = ops.topk_softmax(logits.to(DEV), K_TOP, True)
    assert torch.equal(ti.long(), ti2)
    assert torch.equal(tw, tw2)
    q_ref, s_ref = O.quant_fp8_per_token_group(x, 128)
    assert torch.equal(hq.cpu().float(), q_ref.float())
    assert torch.equal(hs.cpu(), s_ref)


@pytest.mark.parametrize("M,a_mode,ids64", [(32, "q16", False), (32, "bf16", True), (1, "q16", False),
                                            (24, "q16", True), (64, "bf16", True), (7, "bf16", False)])
def test_stream_gemm_decode_layer(M, a_mode, ids64):
    """topk+quant -> gate_up (fused SiLU-and-mul) -> down x routed weight ->
    top-k sum, all through the C-ABI, against the oracle."""
    from mstar_amd import _lib, ops
    q1, s1, q2, s2 = _weights()
    x, logits = _inputs(M, seed=100 + M)
    tw, ti, hq, hs = _route_quant(x, logits)
    ids = ti.long() if ids64 else ti
    slots = M * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, H, dtype=torch.bfloat16, device=DEV)
    if a_mode == "q16":
        _stream_gemm(hq, _lib.DT_FP8_AS_BF16, hs, q1, s1, c2, tw, ids, slots, 2 * I, H, K_TOP, 0, 0)
    else:
        _stream_gemm(x.to(DEV), _lib.DT_BF16, None, q1, s1, c2, tw, ids, slots, 2 * I, H, K_TOP, 0, 0)
    _stream_gemm(c2, _lib.DT_BF16, None, q2, s2, c3, tw, ids, slots, H, I, 1, 1, -1)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum_reduce(c3.view(M, K_TOP, H), out, 1.0)
    ref = _ref(x, tw.cpu(), ti.cpu().long())
    assert_moe_close(out, ref, what=f"stream gemm M={M} A={a_mode}")


@pytest.mark.parametrize("a_mode", ["q16", "bf16"])
def test_stream_gemm_skewed_routing_uses_windows(a_mode):
    """Every token routed to the same 8 experts (128 slots each): each CU's
    staged row set exceeds its LDS budget and is processed in windows."""
    from mstar_amd import _lib, ops
    q1, s1, q2, s2 = _weights()
    M = 128
    x, logits = _inputs(M, seed=5)
    _, _, hq, hs = _route_quant(x, logits)
    g = torch.Generator().manual_seed(6)
    ti = torch.stack([torch.randperm(8, generator=g) for _ in range(M)]).int()
    tw = torch.softmax(torch.randn(M, K_TOP, generator=g), dim=-1)
    slots = M * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, H, dtype=torch.bfloat16, device=DEV)
    twd, tid = tw.to(DEV), ti.to(DEV)
    if a_mode == "q16":
        _stream_gemm(hq, _lib.DT_FP8_AS_BF16, hs, q1, s1, c2, twd, tid, slots, 2 * I, H, K_TOP, 0, 0)
    else:
        _stream_gemm(x.to(DEV), _lib.DT_BF16, None, q1, s1, c2, twd, tid, slots, 2 * I, H, K_TOP, 0, 0)
    _stream_gemm(c2, _lib.DT_BF16, None, q2, s2, c3, twd, tid, slots, H, I, 1, 1, -1)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum_reduce(c3.view(M, K_TOP, H), out, 1.0)
    ref = _ref(x, tw, ti.long())
    assert_moe_close(out, ref, what=f"stream gemm skewed A={a_mode}")


def test_stream_gemm_rejects_widened_rows_beyond_slot_limit():
    """FP8_AS_BF16 activations are served by the router-ids kernel only, for
    at most 1024 slots; beyond that the call says so."""
    from mstar_amd import _lib
    lib = _lib.load()
    st = lib.mstar_moe_stream_gemm(None, _lib.DT_FP8_AS_BF16, None, None, None, None, None,
                                   _lib.DT_F32, None, _lib.DT_I32, 2048, E, 2 * I, H, K_TOP, 0, 0,
                                   None)
    assert st == 1  # invalid argument: num_slots > 1024


def layer_sync_words(num_experts):
    import ctypes
    from mstar_amd import _lib
    n = ctypes.c_int64(0)
    _lib.check(_lib.load().mstar_moe_layer_sync_words(num_experts, ctypes.byref(n)), "layer_sync_words")
    return n.value


def _stream_layer(hq, hs, tw, ti, M, c2, c3, sync=None):
    from mstar_amd import _lib
    lib = _lib.load()
    q1, s1, q2, s2 = _weights()
    if sync is None:
        sync = torch.zeros(layer_sync_words(E), dtype=torch.int32, device=DEV)
    _lib.check(lib.mstar_moe_stream_layer(
        hq.data_ptr(), hs.data_ptr(), q1.data_ptr(), s1.data_ptr(), q2.data_ptr(), s2.data_ptr(),
        tw.data_ptr(), ti.data_ptr(), M, H, E, I, K_TOP, 0, c2.data_ptr(), c3.data_ptr(),
        sync.data_ptr(), _lib.stream_of(hq)), "moe_stream_layer")
    return sync


@pytest.mark.parametrize("M,skewed", [(32, False), (1, False), (64, False), (128, True)])
def test_stream_layer_one_launch(M, skewed):
    """mstar_moe_stream_layer (gate_up and down in one launch, the down work of
    an expert waiting for its gate_up rows) equals the two-launch composition
    bit for bit and the oracle within tolerance.  Skewed: every token on the
    same 8 experts (128 rows each), so both phases stage in windows and every
    down window waits on gate_up work spread over many workgroups."""
    from mstar_amd import _lib, ops
    q1, s1, q2, s2 = _weights()
    x, logits = _inputs(M, seed=300 + M)
    tw, ti, hq, hs = _route_quant(x, logits)
    if skewed:
        g = torch.Generator().manual_seed(7)
        ti = torch.stack([torch.randperm(8, generator=g) for _ in range(M)]).int().to(DEV)
        tw = torch.softmax(torch.randn(M, K_TOP, generator=g), dim=-1).to(DEV)
    slots = M * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, H, dtype=torch.bfloat16, device=DEV)
    sync = _stream_layer(hq, hs, tw, ti, M, c2, c3)
    assert int(sync[E]) == 0, "a down-phase wait gave up"
    c2r = torch.empty_like(c2)
    c3r = torch.empty_like(c3)
    _stream_gemm(hq, _lib.DT_FP8_AS_BF16, hs, q1, s1, c2r, tw, ti, slots, 2 * I, H, K_TOP, 0, 0)
    _stream_gemm(c2r, _lib.DT_BF16, None, q2, s2, c3r, tw, ti, slots, H, I, 1, 1, -1)
    assert torch.equal(c2, c2r)
    assert torch.equal(c3, c3r)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum_reduce(c3.view(M, K_TOP, H), out, 1.0)
    ref = _ref(x, tw.cpu(), ti.cpu().long())
    assert_moe_close(out, ref, what=f"stream layer M={M} skewed={skewed}")


def test_stream_layer_repeated_launches_agree():
    """Twenty launches on fresh sync words give identical rows (the per-expert
    waits order every read after the matching writes on every launch)."""
    x, logits = _inputs(32, seed=77)
    tw, ti, hq, hs = _route_quant(x, logits)
    slots = 32 * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, H, dtype=torch.bfloat16, device=DEV)
    _stream_layer(hq, hs, tw, ti, 32, c2, c3)
    first = c3.clone()
    for _ in range(20):
        c3.fill_(0)
        sync = _stream_layer(hq, hs, tw, ti, 32, c2, c3)
        assert int(sync[E]) == 0
        assert torch.equal(c3, first)


@pytest.mark.parametrize("M", [1, 16, 64])
def test_moe_layer_one_launch_talker_shape(M):
    """The Qwen3-Omni talker MoE shape (hidden 1024, inter 384, 128 experts,
    top-8) through mstar_moe_layer, whose decode sizes run the experts in one
    launch (its lists sit after the larger of the two phases' rings, the
    3-step down ring): equal to the two-launch composition bit for bit and to
    the oracle within tolerance."""
    from mstar_amd import _lib, ops, quant
    Ht, It = 1024, 384
    g = torch.Generator().manual_seed(21)
    w1 = (torch.randn(E, 2 * It, Ht, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E, Ht, It, generator=g) * 0.02).to(DEV)
    q1, s1 = quant.quantize_fp8_block(w1)
    q2, s2 = quant.quantize_fp8_block(w2)
    x = torch.randn(M, Ht, generator=g).to(torch.bfloat16)
    logits = torch.randn(M, E, generator=g)
    out, tw, ti = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, K_TOP, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)
    lib = _lib.load()
    tw2 = torch.empty(M, K_TOP, dtype=torch.float32, device=DEV)
    ti2 = torch.empty(M, K_TOP, dtype=torch.int32, device=DEV)
    hq = torch.empty(M, Ht, dtype=torch.bfloat16, device=DEV)
    hs = torch.empty(M, Ht // 128, dtype=torch.float32, device=DEV)
    xd, ld = x.to(DEV), logits.to(DEV)
    _lib.check(lib.mstar_moe_topk_softmax_quant(
        ld.data_ptr(), _lib.DT_F32, M, E, K_TOP, 1, tw2.data_ptr(), ti2.data_ptr(), None,
        xd.data_ptr(), Ht, hq.data_ptr(), hs.data_ptr(), _lib.stream_of(xd)), "topk_softmax_quant")
    slots = M * K_TOP
    c2 = torch.empty(slots, It, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, Ht, dtype=torch.bfloat16, device=DEV)
    for A, a_dt, a_s, B, b_s, C, N, Kd, tk, mul, act in (
            (hq, _lib.DT_FP8_AS_BF16, hs, q1, s1, c2, 2 * It, Ht, K_TOP, 0, 0),
            (c2, _lib.DT_BF16, None, q2, s2, c3, Ht, It, 1, 1, -1)):
        _lib.check(lib.mstar_moe_stream_gemm(
            A.data_ptr(), a_dt, _lib.ptr(a_s), B.data_ptr(), b_s.data_ptr(), C.data_ptr(),
            tw2.data_ptr(), _lib.DT_F32, ti2.data_ptr(), _lib.DT_I32, slots, E, N, Kd,
            tk, mul, act, _lib.stream_of(A)), "moe_stream_gemm")
    ref2 = torch.empty(M, Ht, dtype=torch.bfloat16, device=DEV)
    ops.moe_sum_reduce(c3.view(M, K_TOP, Ht), ref2, 1.0)
    assert torch.equal(out, ref2)
    rw, rids = O.router_topk_softmax(logits, K_TOP, True)
    ref = O.fused_experts_rounding(x, None, None, rw, rids, w1_dq=O.dequant_fp8_block(q1.cpu(), s1.cpu()),
                                   w2_dq=O.dequant_fp8_block(q2.cpu(), s2.cpu()), act_quant=True)
    assert_moe_close(out, ref, what=f"moe_layer talker M={M}")


def test_layer_wait_failures_stay_zero():
    """No wait of a one-launch layer kernel gives up in normal use."""
    import ctypes
    from mstar_amd import _lib
    lib = _lib.load()
    x, logits = _inputs(32, seed=78)
    tw, ti, hq, hs = _route_quant(x, logits)
    c2 = torch.empty(256, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(256, H, dtype=torch.bfloat16, device=DEV)
    n0 = ctypes.c_int(-1)
    _lib.check(lib.mstar_moe_layer_wait_failures(ctypes.byref(n0)), "moe_layer_wait_failures")
    _stream_layer(hq, hs, tw, ti, 32, c2, c3)
    torch.cuda.synchronize()
    n = ctypes.c_int(-1)
    _lib.check(lib.mstar_moe_layer_wait_failures(ctypes.byref(n)), "moe_layer_wait_failures")
    assert n.value == n0.value


_OPT_OUT_CHILD = r'''
import sys, torch
from mstar_amd import _lib, ops, quant
d = torch.load(sys.argv[1], weights_only=True)
q1, s1, q2, s2 = (d[k].cuda() for k in ("q1", "s1", "q2", "s2"))
out = ops.moe_layer(d["x"].cuda(), d["logits"].cuda(), q1, q2, 8, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)[0]
torch.save({"out": out.cpu()}, sys.argv[2])
'''


def test_one_launch_opt_out_gives_the_same_layer(tmp_path):
    """MSTAR_MOE_ONE_LAUNCH=0 (for callers that run decode layers on several
    streams of one device at once) switches mstar_moe_layer to the two-launch
    form; its output equals the one-launch layer bit for bit."""
    import os
    import subprocess
    import sys
    from mstar_amd import _lib, ops
    q1, s1, q2, s2 = _weights()
    x, logits = _inputs(32, seed=79)
    out = ops.moe_layer(x.to(DEV), logits.to(DEV), q1, q2, K_TOP, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)[0]
    torch.save({"x": x, "logits": logits, "q1": q1.cpu(), "s1": s1.cpu(), "q2": q2.cpu(), "s2": s2.cpu()},
               tmp_path / "in.pt")
    repo = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ, MSTAR_MOE_ONE_LAUNCH="0", PYTHONPATH=repo + os.pathsep + os.environ.get("PYTHONPATH", ""))
    print("child: moe_layer with MSTAR_MOE_ONE_LAUNCH=0", flush=True)
    r = subprocess.run([sys.executable, "-c", _OPT_OUT_CHILD, str(tmp_path / "in.pt"), str(tmp_path / "out.pt")],
                       cwd=repo, env=env, capture_output=True, text=True, timeout=100)
    assert r.returncode == 0, r.stderr[-3000:]
    other = torch.load(tmp_path / "out.pt", weights_only=True)["out"]
    assert torch.equal(out.cpu(), other)


@pytest.mark.parametrize("H_,I_,E_,k_,M", [
    (2048, 768, 64, 4, 33), (2048, 768, 256, 8, 64), (2048, 768, 128, 6, 5),
    (1024, 384, 128, 8, 1), (1024, 384, 64, 4, 64), (1024, 384, 256, 8, 17)])
def test_one_launch_layer_sweep_matches_fused_experts(H_, I_, E_, k_, M):
    """The one-launch decode layer (mstar_moe_layer) at several expert counts,
    top-k and token counts of the thinker and talker shapes equals
    fused_experts (two launches, router ids from the layer) bit for bit, and
    the oracle within tolerance at every point."""
    from mstar_amd import _lib, ops, quant
    from mstar_amd.fused_moe import fused_experts
    g = torch.Generator().manual_seed(H_ + I_ + E_ + k_ + M)
    w1 = (torch.randn(E_, 2 * I_, H_, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E_, H_, I_, generator=g) * 0.02).to(DEV)
    q1, s1 = quant.quantize_fp8_block(w1)
    q2, s2 = quant.quantize_fp8_block(w2)
    x = torch.randn(M, H_, generator=g).to(torch.bfloat16).to(DEV)
    logits = torch.randn(M, E_, generator=g).to(DEV)
    out, tw, ti = ops.moe_layer(x, logits, q1, q2, k_, True, 0, _lib.QUANT_FP8_W8A8, s1, s2)
    ref = fused_experts(x, q1, q2, tw, ti, quant="fp8_w8a8", w1_scale=s1, w2_scale=s2)
    assert torch.equal(out, ref)
    rw, rids = O.router_topk_softmax(logits.cpu(), k_, True)
    oref = O.fused_experts_rounding(x.cpu(), None, None, rw, rids,
                                    w1_dq=O.dequant_fp8_block(q1.cpu(), s1.cpu()),
                                    w2_dq=O.dequant_fp8_block(q2.cpu(), s2.cpu()), act_quant=True)
    assert_moe_close(out, oref, what=f"one-launch layer H={H_} E={E_} k={k_} M={M}")


@pytest.mark.parametrize("quant", ["fp8_w8a8", "w4a16"])
def test_one_launch_layer_gelu(quant):
    """The one-launch decode layer with the GeLU-and-mul gate (activation 1)
    equals fused_experts(activation="gelu") on the layer's own routing bit for
    bit (FP8 and W4A16 weights, M=32 at the thinker shape), and the FP8 layer
    meets the oracle's GeLU layer within tolerance."""
    from mstar_amd import _lib, ops, quant as Q
    from mstar_amd.fused_moe import fused_experts
    H_, I_, E_, k_, M = 2048, 768, 128, 8, 32
    g = torch.Generator().manual_seed(91)
    w1 = (torch.randn(E_, 2 * I_, H_, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E_, H_, I_, generator=g) * 0.02).to(DEV)
    if quant == "fp8_w8a8":
        q1, s1 = Q.quantize_fp8_block(w1)
        q2, s2 = Q.quantize_fp8_block(w2)
        qc = _lib.QUANT_FP8_W8A8
    else:
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        qc = _lib.QUANT_W4A16
    x = torch.randn(M, H_, generator=g).to(torch.bfloat16).to(DEV)
    logits = torch.randn(M, E_, generator=g).to(DEV)
    out, tw, ti = ops.moe_layer(x, logits, q1, q2, k_, True, 1, qc, s1, s2)
    ref = fused_experts(x, q1, q2, tw, ti, "gelu", quant=quant, w1_scale=s1, w2_scale=s2)
    assert torch.equal(out, ref)
    silu, _, _ = ops.moe_layer(x, logits, q1, q2, k_, True, 0, qc, s1, s2)
    assert not torch.equal(out, silu)
    if quant == "fp8_w8a8":
        rw, rids = O.router_topk_softmax(logits.cpu(), k_, True)
        oref = O.fused_experts_rounding(x.cpu(), None, None, rw, rids, activation="gelu",
                                        w1_dq=O.dequant_fp8_block(q1.cpu(), s1.cpu()),
                                        w2_dq=O.dequant_fp8_block(q2.cpu(), s2.cpu()), act_quant=True)
        assert_moe_close(out, oref, what="one-launch layer gelu")


@pytest.mark.parametrize("quant,M", [("w4a16", 64), ("w4a16", 17), ("fp8_w8a8", 64)])
def test_one_launch_layer_skewed_routing(quant, M):
    """Every token routed to the same 8 experts (M rows each): both phases of
    the one-launch layer stage their rows in windows and every down window
    waits on gate_up work of many workgroups.  Bit-exact against
    fused_experts on the same routing, within tolerance of the oracle on that
    routing, and no wait gives up."""
    import ctypes
    from mstar_amd import _lib, ops, quant as Q
    from mstar_amd.fused_moe import fused_experts
    H_, I_, E_, k_ = 2048, 768, 128, 8
    g = torch.Generator().manual_seed(200 + M)
    w1 = (torch.randn(E_, 2 * I_, H_, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E_, H_, I_, generator=g) * 0.02).to(DEV)
    if quant == "fp8_w8a8":
        q1, s1 = Q.quantize_fp8_block(w1)
        q2, s2 = Q.quantize_fp8_block(w2)
        qc = _lib.QUANT_FP8_W8A8
    else:
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        qc = _lib.QUANT_W4A16
    x = torch.randn(M, H_, generator=g).to(torch.bfloat16).to(DEV)
    logits = torch.randn(M, E_, generator=g)
    logits[:, 40:48] += 50.0  # experts 40-47 win for every token
    logits = logits.to(DEV)
    lib = _lib.load()
    before = ctypes.c_int(-1)
    _lib.check(lib.mstar_moe_layer_wait_failures(ctypes.byref(before)), "wait_failures")
    out, tw, ti = ops.moe_layer(x, logits, q1, q2, k_, True, 0, qc, s1, s2)
    assert sorted(set(ti.flatten().tolist())) == list(range(40, 48))
    ref = fused_experts(x, q1, q2, tw, ti, quant=quant, w1_scale=s1, w2_scale=s2)
    assert torch.equal(out, ref)
    c = [t.cpu() for t in (q1, s1, q2, s2)]
    if quant == "fp8_w8a8":
        dq1, dq2 = O.dequant_fp8_block(c[0], c[1]), O.dequant_fp8_block(c[2], c[3])
    else:
        dq1 = lambda e: O.dequant_int4_group(c[0][e], c[1][e])  # noqa: E731
        dq2 = lambda e: O.dequant_int4_group(c[2][e], c[3][e])  # noqa: E731
    oref = O.fused_experts_rounding(x.cpu(), None, None, tw.cpu(), ti.cpu(), w1_dq=dq1, w2_dq=dq2,
                                    act_quant=quant == "fp8_w8a8")
    assert_moe_close(out, oref, what=f"one-launch layer skewed {quant} M={M}")
    torch.cuda.synchronize()
    after = ctypes.c_int(-1)
    _lib.check(lib.mstar_moe_layer_wait_failures(ctypes.byref(after)), "wait_failures")
    assert after.value == before.value
