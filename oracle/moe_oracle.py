"""CPU oracle for the fused-MoE hot path -- TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, what the reference computes on the fused
Mixture-of-Experts path.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and only as the checker
(or as the timed CPU baseline).  The product package ``mstar_amd`` never
imports it: the HIP extension is the only compute path there.

Every function cites the reference file:line it follows (paths relative to
the reference checkout).  Integer work (alignment) is numpy; floating-point
work is PyTorch on the CPU, because the reference's own arithmetic *is*
PyTorch (``torch.softmax``/``torch.topk``/``torch.mm`` bf16 semantics).

Pinning status (how each function is checked by ``tests/test_oracle.py``):

* ``router_topk_softmax`` -- pinned against the closed form
  ``w_i = exp(l_i) / sum_{j in topk} exp(l_j)`` evaluated in float64 with an
  independent numpy argsort, on fixtures asserted to have no near-ties.
* ``moe_align_block_size`` -- pinned bit-exactly against a brute-force
  pure-Python restatement of the CUDA op's contract and against invariants
  (every slot once, ascending within an expert, padding = numel).
* ``naive_dispatch`` -- pinned against a float64 per-token textbook MoE
  ``sum_j w_j W2_e (silu(W1g_e x) * W1u_e x)`` within bf16 tolerance, and
  against the reference test's own bar (fused-rounding vs naive at
  atol=rtol=2e-2).
* ``fused_experts_rounding`` -- pinned against float64 textbook MoE and
  against ``naive_dispatch`` at the reference test's tolerance.
* ``quant_*`` (FP8 e4m3fn, int4) -- pinned against an independent
  pure-Python e4m3fn encoder (enumeration of all 256 codes, round to nearest,
  ties to even), and invariants (the group amax maps to +-448, re-quantising
  a dequantised tensor is idempotent, int4 pack/unpack round trip).
* FP8 / W4A16 MoE and dense FP8 GEMM -- no reference code exists for these
  (the reference stripped them, ``mstar/utils/fused_moe/kernels.py:3-7``);
  they are the reference's bf16 semantics applied to quantise->dequantise
  tensors, pinned against float64 matmuls of the dequantised operands.
"""
from __future__ import annotations

import numpy as np
import math

import torch
import torch.nn.functional as F

FP8_MAX = 448.0
QUANT_EPS = 1e-10


# ---------------------------------------------------------------------------
# a1. Router: softmax top-k (mstar/model/components/moe.py:131-139)
# ---------------------------------------------------------------------------

def router_topk_softmax(logits: torch.Tensor, top_k: int, renormalize: bool = True):
    """Restates ``TopKRouter.forward`` from the logits on.

    moe.py:132  softmax in float32 over experts
    moe.py:135  torch.topk (values sorted descending)
    moe.py:136-137  renormalise by the sum of the selected probabilities
    moe.py:139  cast to the softmax dtype (float32)

    Returns ``(weights fp32 [M,k], ids int64 [M,k])``.

    Ties: ``torch.topk`` leaves the order of equal values unspecified (on the
    CPU it returns tied experts in no fixed order), and equal probabilities
    are common when the router logits are bf16 (``F.linear`` in bf16,
    moe.py:131).  The oracle fixes the rule to "lower expert index first" with
    a stable descending sort; the values equal ``torch.topk``'s.
    """
    probs = F.softmax(logits.float(), dtype=torch.float, dim=-1)
    srt = torch.sort(probs, dim=-1, descending=True, stable=True)
    top_v, top_i = srt.values[..., :top_k], srt.indices[..., :top_k]
    if renormalize:
        top_v = top_v / top_v.sum(dim=-1, keepdim=True)
    return top_v.to(torch.float32), top_i


# ---------------------------------------------------------------------------
# a2. Alignment (mstar/utils/fused_moe/align.py:55-103, 106-152)
# ---------------------------------------------------------------------------

def align_sizes(numel: int, block_size: int, num_experts: int):
    """Buffer sizes chosen by the reference host code (align.py:78-86)."""
    max_padded = numel + num_experts * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    return max_padded, max_blocks


def moe_align_block_size(topk_ids, block_size: int, num_experts: int):
    """Restates ``_moe_align_block_size_torch`` (align.py:106-152) in numpy.

    Returns ``(sorted_token_ids int32, expert_ids int32, ntpp int32[1])``.
    Padding slots hold ``numel`` (align.py:128); unused blocks hold expert 0
    (align.py:129); within an expert, slots keep ascending order -- the
    stable argsort of align.py:146.  Entries ``>= num_experts`` are skipped,
    as the CUDA op does (moe_align_block_size.cu:60-62).
    """
    flat = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    numel = flat.size
    max_padded, max_blocks = align_sizes(numel, block_size, num_experts)
    sorted_ids = np.full(max_padded, numel, dtype=np.int32)
    expert_ids = np.zeros(max_blocks, dtype=np.int32)

    valid = (flat >= 0) & (flat < num_experts)
    counts = np.bincount(flat[valid], minlength=num_experts)[:num_experts]
    padded = ((counts + block_size - 1) // block_size) * block_size
    cumsum = np.zeros(num_experts + 1, dtype=np.int64)
    cumsum[1:] = np.cumsum(padded)
    ntpp = np.array([cumsum[-1]], dtype=np.int32)

    nblocks = padded // block_size
    eidx = np.repeat(np.arange(num_experts, dtype=np.int32), nblocks)
    expert_ids[: eidx.size] = eidx

    slots = np.nonzero(valid)[0]
    order = slots[np.argsort(flat[slots], kind="stable")]
    sorted_e = flat[order]
    ucum = np.zeros(num_experts + 1, dtype=np.int64)
    ucum[1:] = np.cumsum(counts)
    local_rank = np.arange(order.size, dtype=np.int64) - ucum[sorted_e]
    dest = cumsum[sorted_e] + local_rank
    sorted_ids[dest] = order.astype(np.int32)
    return sorted_ids, expert_ids, ntpp


def get_default_config(M: int, E: int):
    """Restates ``get_default_config`` (kernels.py:401-420): the reference's
    block size for the alignment step."""
    if M <= E:
        return {"BLOCK_SIZE_M": 16, "BLOCK_SIZE_N": 32, "BLOCK_SIZE_K": 64, "GROUP_SIZE_M": 1}
    return {"BLOCK_SIZE_M": 64, "BLOCK_SIZE_N": 64, "BLOCK_SIZE_K": 32, "GROUP_SIZE_M": 8}


# ---------------------------------------------------------------------------
# a7. Naive dispatch: the reference CPU path (moe.py:143-185)
# ---------------------------------------------------------------------------

def naive_dispatch(hidden, gate_up_proj, down_proj, num_experts, selected_experts, routing_weights):
    """Restates ``dispatch_experts_fused`` (moe.py:164-185) line by line.

    bf16 ``mm`` per hit expert (ascending expert order), ``F.silu(gate)*up``,
    second ``mm``, multiply by the routing weight (promotes to the weight's
    dtype), cast back, and ``index_add_`` into a zero accumulator of the
    hidden dtype.  This is also the timed CPU baseline.
    """
    final = torch.zeros_like(hidden)
    with torch.no_grad():
        expert_mask = F.one_hot(selected_experts.long(), num_classes=num_experts)
        expert_mask = expert_mask.permute(2, 1, 0)
        expert_hit = torch.greater(expert_mask.sum(dim=(-1, -2)), 0).nonzero()
        for expert_idx_t in expert_hit:
            e = expert_idx_t[0]
            top_k_pos, token_idx = torch.where(expert_mask[e])
            cur = hidden[token_idx]
            gate_up = torch.mm(cur, gate_up_proj[e].T)
            gate, up = gate_up.chunk(2, dim=-1)
            h = torch.mm(F.silu(gate) * up, down_proj[e].T)
            h = h * routing_weights[token_idx, top_k_pos, None]
            final.index_add_(0, token_idx, h.to(final.dtype))
    return final


# ---------------------------------------------------------------------------
# a3-a6. Fused path with the kernels' rounding points
# ---------------------------------------------------------------------------

def _bf(x: torch.Tensor, dtype=torch.bfloat16) -> torch.Tensor:
    return x.to(dtype)


def silu_and_mul_rounded(gate: torch.Tensor, up: torch.Tensor, activation: str = "silu"):
    """Restates ``act_and_mul_kernel`` (kernels.py:265-276) and
    ``_apply_activation`` (kernels.py:231-241): the activation in fp32,
    cast to the input dtype, multiplied by ``up``, stored in the output
    dtype."""
    dt = gate.dtype
    g = gate.float()
    if activation == "silu":
        a = g * torch.sigmoid(g)
    elif activation == "gelu":
        k = 0.7978845608028654
        a = 0.5 * g * (1.0 + (2.0 * torch.sigmoid(2.0 * (k * (g + 0.044715 * g * g * g))) - 1.0))
    else:
        raise ValueError(f"unsupported activation {activation}")
    return (a.to(dt).float() * up.float()).to(dt)


def moe_sum_reduce(cache3: torch.Tensor, routed_scaling_factor: float = 1.0):
    """Restates ``moe_sum_reduce_kernel`` (kernels.py:340-355): fp32 sum over
    the top-k dim, times the scaling factor, cast to the input dtype."""
    return (cache3.float().sum(dim=1) * routed_scaling_factor).to(cache3.dtype)


def fused_experts_rounding(hidden, w1, w2, topk_weights, topk_ids, activation="silu",
                           reduce_results=True, w1_dq=None, w2_dq=None, act_quant=False):
    """Restates ``fused_experts`` (runner.py:88-159) with the kernel rounding
    points: GEMM1 fp32 accumulate -> store in the compute dtype
    (kernels.py:112-138); activation (kernels.py:265-276); GEMM2 fp32
    accumulate, times the routed weight in fp32, store (kernels.py:129-138);
    fp32 top-k sum (kernels.py:340-355).

    ``w1_dq``/``w2_dq`` optionally supply dequantised weights (FP8 / int4
    variants) as a tensor or as a callable ``e -> [N, K]`` evaluated only for
    hit experts; ``act_quant`` applies per-token-group-128 FP8 Q/DQ to both
    GEMM inputs (the W8A8 block-scaled variant).
    """
    def expert(w, dq, e):
        if dq is None:
            return w[e].float()
        return (dq(e) if callable(dq) else dq[e]).float()

    M, H = hidden.shape
    k = topk_ids.shape[1]
    dt = hidden.dtype
    ids = topk_ids.reshape(-1).long()
    tw = topk_weights.reshape(-1).float()
    hit = torch.unique(ids).tolist()
    W1 = {e: expert(w1, w1_dq, e) for e in hit}
    I = W1[hit[0]].shape[0] // 2
    if act_quant:
        q, s = quant_fp8_per_token_group(hidden, 128)
        xa = dequant_fp8_group(q, s, 128)
    else:
        xa = hidden.float()
    slots = M * k
    cache1 = torch.empty(slots, 2 * I, dtype=dt)
    for e in hit:
        sl = torch.nonzero(ids == e).flatten()
        cache1[sl] = _bf(xa[sl // k] @ W1[e].T, dt)
    del W1
    cache2 = silu_and_mul_rounded(cache1[:, :I], cache1[:, I:], activation)
    if act_quant:
        q2, s2 = quant_fp8_per_token_group(cache2, 128)
        a2 = dequant_fp8_group(q2, s2, 128)
    else:
        a2 = cache2.float()
    cache3 = torch.empty(slots, H, dtype=dt)
    for e in hit:
        sl = torch.nonzero(ids == e).flatten()
        cache3[sl] = _bf((a2[sl] @ expert(w2, w2_dq, e).T) * tw[sl, None], dt)
    cache3 = cache3.view(M, k, H)
    if not reduce_results:
        return cache3
    return moe_sum_reduce(cache3)


def textbook_moe_f64(hidden, W1, W2, topk_weights, topk_ids, activation="silu"):
    """Float64 textbook MoE, ``sum_j w_j W2_e (act(W1g_e x) * W1u_e x)`` per
    token, with no intermediate rounding.  Used only to pin the other
    restatements."""
    x = hidden.double()
    W1 = W1.double()
    W2 = W2.double()
    I = W2.shape[2]
    out = torch.zeros(x.shape[0], W2.shape[1], dtype=torch.float64)
    for t in range(x.shape[0]):
        for j in range(topk_ids.shape[1]):
            e = int(topk_ids[t, j])
            gu = W1[e] @ x[t]
            g, u = gu[:I], gu[I:]
            if activation == "silu":
                a = g * torch.sigmoid(g)
            else:
                kk = 0.7978845608028654
                a = 0.5 * g * (1.0 + torch.tanh(kk * (g + 0.044715 * g ** 3)))
            out[t] += float(topk_weights[t, j]) * (W2[e] @ (a * u))
    return out


# ---------------------------------------------------------------------------
# Quantisation formats (no reference code exists)
# ---------------------------------------------------------------------------

def _fp8(x: torch.Tensor) -> torch.Tensor:
    return x.clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)


def quant_fp8_per_token_group(x: torch.Tensor, group: int = 128):
    """Per-token-group FP8: for each row and each run of ``group`` columns,
    ``s = max(amax, eps) / 448`` (fp32) and ``q = e4m3fn(clamp(x / s))``.
    Returns ``(q [rows, cols] e4m3fn, s [rows, cols/group] fp32)``."""
    rows, cols = x.shape
    assert cols % group == 0
    xf = x.float().view(rows, cols // group, group)
    amax = xf.abs().amax(dim=-1).clamp_min(QUANT_EPS)
    s = amax / FP8_MAX
    q = _fp8(xf / s[..., None]).view(rows, cols)
    return q, s.contiguous()


def dequant_fp8_group(q, s, group=128):
    rows, cols = q.shape
    return (q.float().view(rows, cols // group, group) * s[..., None]).view(rows, cols)


def quant_fp8_block(w: torch.Tensor, block=(128, 128)):
    """Weight FP8 with one scale per ``block`` tile of the last two dims:
    ``s = max(amax_tile, eps) / 448``.  ``w`` is ``[..., N, K]``; returns
    ``(q e4m3fn [..., N, K], s fp32 [..., ceil(N/bn), ceil(K/bk)])``."""
    bn, bk = block
    *lead, N, K = w.shape
    nb, kb = -(-N // bn), -(-K // bk)
    wf = torch.zeros(*lead, nb * bn, kb * bk, dtype=torch.float32)
    wf[..., :N, :K] = w.float()
    t = wf.view(*lead, nb, bn, kb, bk)
    amax = t.abs().amax(dim=(-3, -1)).clamp_min(QUANT_EPS)
    s = amax / FP8_MAX
    q = _fp8(t / s[..., :, None, :, None]).view(*lead, nb * bn, kb * bk)[..., :N, :K]
    return q.contiguous(), s.contiguous()


def dequant_fp8_block(q, s, block=(128, 128)):
    bn, bk = block
    N, K = q.shape[-2], q.shape[-1]
    sf = s.repeat_interleave(bn, dim=-2)[..., :N, :].repeat_interleave(bk, dim=-1)[..., :K]
    return q.float() * sf


def quant_fp8_per_row(x: torch.Tensor):
    """Per-token (activations) or per-output-channel (weights) FP8:
    ``s[r] = max(amax_row, eps) / 448``."""
    xf = x.float()
    s = xf.abs().amax(dim=-1).clamp_min(QUANT_EPS) / FP8_MAX
    return _fp8(xf / s[..., None]), s.contiguous()


def fp8_scaled_mm(a_q, a_s, w_q, w_s, out_dtype=torch.bfloat16):
    """``y = bf16((A_q . W_q^T) * s_a[m] * s_w[n])`` with an fp32 accumulator
    (the reference's dense layers are ``F.linear``,
    mstar/model/components/distributed/linear.py:101,412)."""
    acc = a_q.float() @ w_q.float().T
    return (acc * a_s[:, None] * w_s[None, :]).to(out_dtype)


def _ceil_5_significant_bits(x: float) -> float:
    """Smallest value >= x (x > 0) with five significant binary digits, by
    frexp: x = m * 2^e, m in [0.5, 1); keep ceil(m * 32) / 32."""
    m, e = math.frexp(x)
    return math.ldexp(math.ceil(m * 32.0) / 32.0, e)


def quant_int4_group(w: torch.Tensor, group: int = 128):
    """Symmetric int4, one bf16 scale per ``group`` along K:
    ``s = ceil_5bits(max(amax, eps) / 7)`` (five significant bits, exact in
    bf16), ``q = round_half_even(w / s)`` (|q| <= 7 since s >= amax/7).
    Packing: nibble ``u = q + 8``; element ``k`` sits in bits ``4*(k % 8)``
    of int32 word ``k // 8`` (little-endian nibble order).  ``w`` is
    ``[..., N, K]``; returns ``(packed int32 [..., N, K/8], scales bf16
    [..., N, K/group])``."""
    *lead, N, K = w.shape
    assert K % group == 0 and K % 8 == 0
    wf = w.float().view(*lead, N, K // group, group)
    amax = wf.abs().amax(dim=-1).clamp_min(QUANT_EPS)
    q7 = (amax.double() / 7.0).float()  # the fp32 quotient, correctly rounded
    s = torch.tensor([_ceil_5_significant_bits(v) for v in q7.flatten().tolist()],
                     dtype=torch.float32).view(q7.shape).to(torch.bfloat16)
    q = torch.round(wf / s.float()[..., None]).clamp(-8, 7).to(torch.int64).view(*lead, N, K)
    u = (q + 8).view(*lead, N, K // 8, 8)
    shifts = torch.arange(8, dtype=torch.int64) * 4
    packed = (u << shifts).sum(dim=-1)
    packed = torch.where(packed >= 2 ** 31, packed - 2 ** 32, packed).to(torch.int32)
    return packed.contiguous(), s.contiguous()


def unpack_int4(packed: torch.Tensor):
    """Inverse of the packing in :func:`quant_int4_group`; returns q in
    [-8, 7] as int64 ``[..., N, K]``."""
    p = packed.to(torch.int64) & 0xFFFFFFFF
    shifts = torch.arange(8, dtype=torch.int64) * 4
    u = (p[..., None] >> shifts) & 0xF
    return (u - 8).reshape(*packed.shape[:-1], packed.shape[-1] * 8)


def dequant_int4_group(packed, scales, group=128):
    """``w = bf16(q * s)`` -- the bf16 weight the W4A16 GEMM multiplies (exact:
    ``q * s`` needs at most eight significant bits)."""
    q = unpack_int4(packed).float()
    s = scales.float().repeat_interleave(group, dim=-1)
    return (q * s).to(torch.bfloat16)


# ---------------------------------------------------------------------------
# Seeded BASELINE inputs
# ---------------------------------------------------------------------------

def zipf_bias(E: int) -> torch.Tensor:
    """Per-expert router bias of config 3: ``b_e = 2*log(1/(e+1)^1.2)``."""
    e = torch.arange(E, dtype=torch.float64)
    return (2.0 * torch.log(1.0 / (e + 1.0) ** 1.2)).to(torch.float32)


def make_moe_inputs(M, H, E, k, I, seed=0, bias=False, dtype=torch.bfloat16):
    """Seeded synthetic tensors in the order the BASELINE configs list them:
    hidden ~N(0,1), w1 [E,2I,H] and w2 [E,H,I] ~N(0,0.02), logits [M,E]
    ~N(0,1) (fp32), plus the Zipf bias when ``bias``."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, H, generator=g).to(dtype)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(dtype)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(dtype)
    logits = torch.randn(M, E, generator=g)
    if bias:
        logits = logits + zipf_bias(E)[None, :]
    return x, w1, w2, logits
