"""Pin the CPU oracle (oracle/moe_oracle.py) against independent checks.

No reference test ships golden vectors for this path (the reference's MoE
test compares fused vs naive in one process,
test/modular/test_qwen3_omni_fused_moe.py:71-102), so each oracle function is
checked against something it does not share code with: brute force, closed
forms evaluated another way, float64 textbook math, or an independent
bit-level encoder.  Runs on the CPU.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe_oracle as O
from tests._util import align_brute_force, assert_moe_close

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ----------------------------------------------------------------- alignment
ALIGN_CASES = [
    # (numel-shape, E, block, kind)
    ((64, 2), 8, 64, "uniform"),     # C1 tiny: M=64 > E=8 -> BM=64
    ((32, 8), 128, 16, "uniform"),   # C2 decode: BM=16
    ((1, 8), 128, 16, "uniform"),
    ((5, 3), 4, 1, "uniform"),
    ((7, 2), 1, 4, "uniform"),       # single expert
    ((40, 4), 16, 8, "skewed"),      # most slots to expert 0
    ((33, 2), 8, 16, "invalid"),     # ids >= E are skipped
    ((0, 8), 128, 16, "uniform"),    # empty
    ((300, 8), 128, 64, "zipf"),
]


def _ids(shape, E, kind, seed):
    g = torch.Generator().manual_seed(seed)
    if kind == "uniform":
        return torch.randint(0, E, shape, generator=g)
    if kind == "skewed":
        x = torch.randint(0, E, shape, generator=g)
        x[torch.rand(shape, generator=g) < 0.7] = 0
        return x
    if kind == "invalid":
        return torch.randint(0, E + 3, shape, generator=g)
    if kind == "zipf":
        logits = torch.randn(shape[0], E, generator=g) + O.zipf_bias(E)
        return torch.topk(logits, shape[1], dim=-1).indices
    raise ValueError(kind)


@pytest.mark.parametrize("shape,E,bm,kind", ALIGN_CASES)
def test_align_matches_brute_force(shape, E, bm, kind):
    ids = _ids(shape, E, kind, seed=hash((shape, E, bm, kind)) % 1000)
    s, e, n = O.moe_align_block_size(ids.numpy(), bm, E)
    bs, be, bn = align_brute_force(ids, bm, E)
    assert s.tolist() == bs
    assert e.tolist() == be
    assert int(n[0]) == bn


def test_align_invariants_prefill_shape():
    # C3 prefill at M=8192, top-8, Zipf-biased: every valid slot exactly once,
    # ascending inside each expert, padding == numel, blocks of one expert.
    ids = _ids((8192, 8), 128, "zipf", seed=3)
    bm = 64
    s, e, n = O.moe_align_block_size(ids.numpy(), bm, 128)
    numel = ids.numel()
    ntpp = int(n[0])
    assert ntpp % bm == 0
    real = s[:ntpp][s[:ntpp] < numel]
    assert np.array_equal(np.sort(real), np.arange(numel))
    flat = ids.reshape(-1).numpy()
    for b in range(ntpp // bm):
        blk = s[b * bm:(b + 1) * bm]
        v = blk[blk < numel]
        assert (flat[v] == e[b]).all()
        assert (np.diff(v) > 0).all()
    assert (s[ntpp:] == numel).all()


# ------------------------------------------------------------------- router
def _router_closed_form(logits: torch.Tensor, k: int, renorm: bool):
    """ids = the k largest logits (softmax is monotonic); weights
    exp(l_i - m) / sum_{selected or all} exp(l_j - m) in float64."""
    L = logits.double().numpy()
    ids = np.argsort(-L, axis=-1, kind="stable")[:, :k]
    m = L.max(axis=-1, keepdims=True)
    ex = np.exp(L - m)
    sel = np.take_along_axis(ex, ids, axis=-1)
    den = sel.sum(-1, keepdims=True) if renorm else ex.sum(-1, keepdims=True)
    return ids, sel / den


def _min_topk_gap(logits: torch.Tensor, k: int) -> float:
    srt = torch.sort(logits.double(), dim=-1, descending=True).values
    return float((srt[:, k - 1] - srt[:, k]).min())


@pytest.mark.parametrize("M,E,k,bias,renorm", [
    (64, 8, 2, False, True),       # C1
    (32, 128, 8, False, True),     # C2
    (512, 128, 8, True, True),     # C3 (M=512 of the sweep)
    (16, 128, 8, False, False),    # talker: norm_topk_prob=False
])
def test_router_closed_form(M, E, k, bias, renorm):
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(M, E, generator=g)
    if bias:
        logits = logits + O.zipf_bias(E)
    assert _min_topk_gap(logits, k) > 1e-6  # no near-ties at the selection boundary
    w, ids = O.router_topk_softmax(logits, k, renorm)
    cids, cw = _router_closed_form(logits, k, renorm)
    assert np.array_equal(ids.numpy(), cids)
    assert np.allclose(w.double().numpy(), cw, rtol=2e-6, atol=1e-9)
    assert w.dtype == torch.float32 and ids.dtype == torch.int64


def test_router_matches_reference_test_construction():
    # The reference test builds its router output as softmax -> topk ->
    # renormalise (test/modular/test_qwen3_omni_fused_moe.py:32-49).
    g = torch.Generator().manual_seed(1)
    logits = torch.randn(16, 128, generator=g)
    probs = torch.softmax(logits, dim=-1)
    tw, ti = torch.topk(probs, 8, dim=-1)
    tw = tw / tw.sum(dim=-1, keepdim=True)
    w, ids = O.router_topk_softmax(logits, 8, True)
    assert torch.equal(ids, ti)
    assert torch.equal(w, tw)


def test_router_tie_rule_keeps_topk_values():
    # bf16 logits tie often; the oracle's order is lower index first and its
    # values are exactly torch.topk's.
    g = torch.Generator().manual_seed(2)
    logits = torch.randn(500, 128, generator=g).to(torch.bfloat16).float()
    logits[0, [3, 5, 9]] = 4.0
    w, ids = O.router_topk_softmax(logits, 8, False)
    tv, _ = torch.topk(torch.softmax(logits, -1), 8, dim=-1)
    assert torch.equal(w, tv)
    assert ids[0, :3].tolist() == [3, 5, 9]
    L = logits.double().numpy()
    assert np.array_equal(ids.numpy(), np.argsort(-L, axis=-1, kind="stable")[:, :8])


def test_zipf_bias_formula():
    b = O.zipf_bias(4)
    for e in range(4):
        assert math.isclose(float(b[e]), 2 * math.log(1 / (e + 1) ** 1.2), rel_tol=1e-6)


# ----------------------------------------------------------- MoE arithmetic
def _small_moe(M=24, H=128, E=6, k=2, I=128, seed=0, dtype=torch.bfloat16):
    x, w1, w2, logits = O.make_moe_inputs(M, H, E, k, I, seed=seed, dtype=dtype)
    tw, ti = O.router_topk_softmax(logits, k, True)
    return x, w1, w2, tw, ti


def test_naive_dispatch_vs_textbook():
    x, w1, w2, tw, ti = _small_moe()
    out = O.naive_dispatch(x, w1, w2, w1.shape[0], ti, tw)
    ref = O.textbook_moe_f64(x.float(), w1.float(), w2.float(), tw, ti)
    assert out.dtype == torch.bfloat16
    assert_moe_close(out, ref, max_rel=2e-2, mean_of_rms=1e-2, what="naive vs f64")


def test_fused_rounding_vs_textbook_and_naive():
    x, w1, w2, tw, ti = _small_moe(seed=1)
    fused = O.fused_experts_rounding(x, w1, w2, tw, ti)
    ref = O.textbook_moe_f64(x.float(), w1.float(), w2.float(), tw, ti)
    assert_moe_close(fused, ref, max_rel=2e-2, mean_of_rms=1e-2, what="fused vs f64")
    naive = O.naive_dispatch(x, w1, w2, w1.shape[0], ti, tw)
    # The reference test's own bar (test_qwen3_omni_fused_moe.py:102).
    torch.testing.assert_close(fused, naive, atol=2e-2, rtol=2e-2)


def test_fused_rounding_gelu_and_unreduced():
    x, w1, w2, tw, ti = _small_moe(seed=2)
    out3 = O.fused_experts_rounding(x, w1, w2, tw, ti, activation="gelu", reduce_results=False)
    assert out3.shape == (x.shape[0], ti.shape[1], x.shape[1])
    ref = O.textbook_moe_f64(x.float(), w1.float(), w2.float(), tw, ti, activation="gelu")
    assert_moe_close(O.moe_sum_reduce(out3), ref, max_rel=2e-2, mean_of_rms=1e-2)


def test_silu_and_mul_rounding_points():
    g = torch.tensor([0.0, 1.0, -3.5, 10.0], dtype=torch.bfloat16)
    u = torch.tensor([2.0, -1.0, 0.5, 1.0], dtype=torch.bfloat16)
    out = O.silu_and_mul_rounded(g, u)
    expect = [0.0, -float(F.silu(torch.tensor(1.0)).to(torch.bfloat16)),
              float((F.silu(torch.tensor(-3.5)).to(torch.bfloat16).float() * 0.5).to(torch.bfloat16)),
              float(F.silu(torch.tensor(10.0)).to(torch.bfloat16))]
    assert out.float().tolist() == expect


def test_sum_reduce_scaling():
    x = torch.randn(3, 4, 16).to(torch.bfloat16)
    out = O.moe_sum_reduce(x, 0.5)
    assert torch.equal(out, (x.double().sum(1) * 0.5).to(torch.bfloat16))


# ------------------------------------------------------------------ FP8 e4m3
def _e4m3fn_values():
    """All 256 e4m3fn codes decoded from the OCP definition (bias 7,
    subnormals at exponent 0, S.1111.111 is NaN, no infinities)."""
    vals = []
    for c in range(256):
        s = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            vals.append(float("nan"))
        elif e == 0:
            vals.append(s * (m / 8.0) * 2.0 ** -6)
        else:
            vals.append(s * (1.0 + m / 8.0) * 2.0 ** (e - 7))
    return vals


def _encode_e4m3fn(x: float) -> float:
    """Round to nearest representable e4m3fn, ties to the even code,
    saturating inputs beyond 448 is the caller's job (we clamp first)."""
    vals = [v for v in _e4m3fn_values() if not math.isnan(v)]
    codes = [c for c, v in enumerate(_e4m3fn_values()) if not math.isnan(v)]
    best = None
    for c, v in zip(codes, vals):
        d = abs(v - x)
        if best is None or d < best[0] - 0.0 or (d == best[0] and (c & 1) == 0 and (best[1] & 1)):
            best = (d, c, v)
    return best[2]


def test_fp8_conversion_matches_independent_encoder():
    vals = torch.tensor([v for v in _e4m3fn_values() if not math.isnan(v)])
    # Every representable value and every midpoint between neighbours.
    pos = torch.unique(vals.abs())
    mids = (pos[1:] + pos[:-1]) / 2
    g = torch.Generator().manual_seed(0)
    probe = torch.cat([pos, mids, -mids, torch.rand(200, generator=g) * 448,
                       torch.randn(200, generator=g) * 3, torch.tensor([1e-9, -1e-9, 447.9])])
    got = O._fp8(probe).float()
    exp = torch.tensor([_encode_e4m3fn(float(v)) for v in probe.clamp(-448, 448)])
    assert torch.equal(got, exp)


def test_fp8_group_quant_invariants():
    g = torch.Generator().manual_seed(0)
    x = (torch.randn(8, 512, generator=g) * 3).to(torch.bfloat16)
    x[0, :128] = 0  # all-zero group: eps scale, zero codes
    q, s = O.quant_fp8_per_token_group(x, 128)
    assert q.dtype == torch.float8_e4m3fn and s.shape == (8, 4)
    qf = q.float().view(8, 4, 128)
    assert (qf[0, 0] == 0).all()
    nz = qf.abs().amax(-1)[1:]
    assert (nz == 448).all()  # the group maximum lands exactly on the top code
    xf = x.float().view(8, 4, 128)
    err = (qf * s[..., None] - xf).abs()
    # Half a step at the value's binade: e4m3 has 3 mantissa bits.
    bound = (xf.abs() / 16 + 2.0 ** -10 * s[..., None]) + 1e-12
    assert (err <= bound * 1.0001 + s[..., None] * 2.0 ** -9).all()
    # Re-quantising the dequantised tensor reproduces the same codes.
    q2, s2 = O.quant_fp8_per_token_group(O.dequant_fp8_group(q, s, 128), 128)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8))


def test_fp8_block_quant_matches_group_rule():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(2, 256, 384, generator=g) * 0.02
    q, s = O.quant_fp8_block(w)
    assert s.shape == (2, 2, 3)
    for e in range(2):
        for nb in range(2):
            for kb in range(3):
                t = w[e, nb * 128:(nb + 1) * 128, kb * 128:(kb + 1) * 128]
                assert float(s[e, nb, kb]) == float(torch.tensor(float(t.abs().max()) / 448.0, dtype=torch.float32))
    dq = O.dequant_fp8_block(q, s)
    assert ((dq - w).abs() <= w.abs() / 16 + 1e-6).all()


def test_fp8_scaled_mm_vs_f64():
    g = torch.Generator().manual_seed(0)
    a = torch.randn(16, 256, generator=g).to(torch.bfloat16)
    w = torch.randn(48, 256, generator=g) * 0.02
    aq, as_ = O.quant_fp8_per_row(a)
    wq, ws = O.quant_fp8_per_row(w)
    out = O.fp8_scaled_mm(aq, as_, wq, ws)
    ref = (aq.double() * as_.double()[:, None]) @ (wq.double() * ws.double()[:, None]).T
    assert_moe_close(out, ref, max_rel=1e-2, mean_of_rms=3e-3)
    # ... and the quantisation itself stays within FP8 error of the bf16 product.
    full = a.double() @ w.double().T
    assert_moe_close(out, full, max_rel=8e-2, mean_of_rms=5e-2)


# ------------------------------------------------------------------- int4
def test_int4_pack_roundtrip_and_layout():
    g = torch.Generator().manual_seed(0)
    w = torch.randn(3, 8, 256, generator=g) * 0.02
    packed, s = O.quant_int4_group(w, 128)
    assert packed.shape == (3, 8, 32) and s.shape == (3, 8, 2) and s.dtype == torch.bfloat16
    q = O.unpack_int4(packed)
    assert q.min() >= -8 and q.max() <= 7
    # Independent nibble read-back for one word: element k at bits 4*(k%8).
    word = int(packed[1, 2, 5]) & 0xFFFFFFFF
    for n in range(8):
        assert ((word >> (4 * n)) & 0xF) - 8 == int(q[1, 2, 5 * 8 + n])
    # Scale: the first value >= amax/7 with five significant bits (checked
    # by brute force over the 16 five-bit mantissas of amax/7's binade).
    amax = w.view(3, 8, 2, 128).abs().amax(dim=-1)
    for a_, s_ in zip(amax.flatten().tolist(), s.float().flatten().tolist()):
        t = a_ / 7.0
        e = math.floor(math.log2(t))
        cands = [(16 + i) / 16.0 * 2.0 ** e for i in range(17)]
        assert s_ == min(c for c in cands if c >= t)
    # Symmetric rounding: q = round(w / s), |q| <= 7.
    sf = s.float().repeat_interleave(128, dim=-1)
    assert torch.equal(q.float(), torch.round(w / sf))
    assert q.abs().max() <= 7
    dq = O.dequant_int4_group(packed, s)
    # q*s is exact in bf16 (so kernels may scale after the dot product) ...
    assert torch.equal(dq.double(), q.double() * sf.double())
    # ... and within half a step of w.
    assert ((dq.float() - w).abs() <= sf / 2 + 1e-12).all()


def test_quantised_moe_oracle_vs_textbook():
    # FP8 W8A8: the rounding-point oracle on Q/DQ tensors agrees with f64
    # textbook math on the same dequantised weights and activations.
    x, w1, w2, tw, ti = _small_moe(H=256, I=256, seed=4)
    q1, s1 = O.quant_fp8_block(w1)
    q2, s2 = O.quant_fp8_block(w2)
    d1, d2 = O.dequant_fp8_block(q1, s1), O.dequant_fp8_block(q2, s2)
    out = O.fused_experts_rounding(x, None, None, tw, ti, w1_dq=d1, w2_dq=d2, act_quant=True)
    xq, xs = O.quant_fp8_per_token_group(x, 128)
    ref = O.textbook_moe_f64(O.dequant_fp8_group(xq, xs), d1, d2, tw, ti)
    assert_moe_close(out, ref, max_rel=5e-2, mean_of_rms=3e-2)
    # W4A16
    p1, t1 = O.quant_int4_group(w1)
    p2, t2 = O.quant_int4_group(w2)
    e1, e2 = O.dequant_int4_group(p1, t1), O.dequant_int4_group(p2, t2)
    out4 = O.fused_experts_rounding(x, e1, e2, tw, ti)
    ref4 = O.textbook_moe_f64(x.float(), e1.float(), e2.float(), tw, ti)
    assert_moe_close(out4, ref4, max_rel=2e-2, mean_of_rms=1e-2)


# ------------------------------------------------------------- golden files
def test_golden_fixtures_reproduce():
    """The committed fixtures (tests/golden/*.npz) are what the oracle
    computes today -- guards against silent oracle drift."""
    from tests.golden import make_golden
    files = [f for f in os.listdir(GOLDEN) if f.endswith(".npz")]
    assert files, "no golden fixtures committed"
    for f in files:
        data = np.load(os.path.join(GOLDEN, f), allow_pickle=False)
        fresh = make_golden.compute(f[:-4])
        for key in data.files:
            assert np.array_equal(data[key], fresh[key]), (f, key)
