"""torch.library custom ops over the C-ABI.

Each op launches on the calling thread's current stream of the input's
device, allocates its outputs (and any workspace) through PyTorch's caching
allocator, and has a fake (meta) implementation so ``torch.compile`` can trace
it and HIP-graph capture sees static shapes -- the two conditions the
reference's capture path imposes (mstar/engine/cuda_graph_runner.py:617-640).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

from . import _lib
from ._lib import check, dtype_code, load, ptr, stream_of

_NS = "mstar_moe"


def _wait_checks_on() -> bool:
    return os.environ.get("MSTAR_MOE_CHECK_WAITS", "0") not in ("", "0") and \
        not torch.cuda.is_current_stream_capturing()


def _layer_wait_failures() -> int:
    n = ctypes.c_int(0)
    check(load().mstar_moe_layer_wait_failures(ctypes.byref(n)), "moe_layer_wait_failures")
    return n.value


def _check_layer_waits(what: str) -> None:
    """With MSTAR_MOE_CHECK_WAITS=1 in the environment (read per call), an
    eager layer call synchronises and raises if a wait of the one-launch
    decode layer kernel gave up during it (its output rows are then NaN);
    under stream capture there is nothing to read, and the check is skipped.
    Off by default: it costs a device synchronisation per call."""
    if not _wait_checks_on():
        return
    torch.cuda.synchronize()
    n = _layer_wait_failures()
    dev = torch.cuda.current_device()
    seen = _WAIT_FAILURES.get(dev, n)
    _WAIT_FAILURES[dev] = n
    if n > seen:
        raise _lib.MstarError(f"{what}: {n - seen} wait(s) of the one-launch decode layer gave up "
                              "(its output is invalid; see mstar_moe_layer_wait_failures)")


_WAIT_FAILURES: dict = {}


def _on_device(fn):
    """Run an op with its first tensor argument's device current, as the
    reference's OptionalCUDAGuard does (moe_align_block_size.cu:213): the
    launchers size grids and LDS for the current device, and the kernels go
    to that device's current stream."""
    import functools

    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        for a in args:
            if isinstance(a, torch.Tensor) and a.is_cuda:
                with torch.cuda.device(a.device):
                    return fn(*args, **kwargs)
        return fn(*args, **kwargs)

    return wrapper


def _act_code(activation: str) -> int:
    if activation == "silu":
        return 0
    if activation == "gelu":
        return 1
    raise ValueError(f"unsupported activation {activation!r}; use 'silu' or 'gelu'")


# ------------------------------------------------------------------ routing
@torch.library.custom_op(f"{_NS}::topk_softmax", mutates_args=())
@_on_device
def topk_softmax(logits: torch.Tensor, top_k: int, renormalize: bool) -> tuple[torch.Tensor, torch.Tensor]:
    _lib.require_gpu(logits)
    logits = logits.contiguous()
    M, E = logits.shape
    w = torch.empty(M, top_k, dtype=torch.float32, device=logits.device)
    ids = torch.empty(M, top_k, dtype=torch.int64, device=logits.device)
    check(load().mstar_moe_topk_softmax(ptr(logits), dtype_code(logits.dtype), M, E, top_k,
                                        int(renormalize), ptr(w), None, ptr(ids), stream_of(logits)),
          "topk_softmax")
    return w, ids


@topk_softmax.register_fake
def _(logits, top_k, renormalize):
    M = logits.shape[0]
    return (logits.new_empty(M, top_k, dtype=torch.float32),
            logits.new_empty(M, top_k, dtype=torch.int64))


@torch.library.custom_op(f"{_NS}::router", mutates_args=())
@_on_device
def router(hidden: torch.Tensor, gate_weight: torch.Tensor, top_k: int,
           renormalize: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """TopKRouter.forward (moe.py:114-140) in one launch: bf16 logits =
    hidden . gate_weight^T, fp32 softmax, top-k, optional renormalisation.
    Returns (weights fp32 [T, k], ids int64 [T, k])."""
    _lib.require_gpu(hidden)
    hidden = hidden.reshape(-1, hidden.shape[-1]).contiguous()
    gate_weight = gate_weight.contiguous()
    if hidden.dtype != torch.bfloat16 or gate_weight.dtype != torch.bfloat16:
        raise ValueError("router: hidden states and gate weight must be bfloat16")
    M, H = hidden.shape
    E = gate_weight.shape[0]
    if gate_weight.shape[1] != H:
        raise ValueError(f"router: gate weight {tuple(gate_weight.shape)} does not match hidden size {H}")
    w = torch.empty(M, top_k, dtype=torch.float32, device=hidden.device)
    ids = torch.empty(M, top_k, dtype=torch.int64, device=hidden.device)
    check(load().mstar_moe_router(ptr(hidden), dtype_code(hidden.dtype), M, H, ptr(gate_weight), E,
                                  top_k, int(renormalize), ptr(w), None, ptr(ids), None,
                                  stream_of(hidden)), "router")
    return w, ids


@router.register_fake
def _(hidden, gate_weight, top_k, renormalize):
    M = hidden.numel() // hidden.shape[-1]
    return (hidden.new_empty(M, top_k, dtype=torch.float32),
            hidden.new_empty(M, top_k, dtype=torch.int64))


@torch.library.custom_op(f"{_NS}::moe_align_block_size", mutates_args=())
@_on_device
def moe_align_block_size(topk_ids: torch.Tensor, block_size: int,
                         num_experts: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _lib.require_gpu(topk_ids)
    topk_ids = topk_ids.contiguous()
    numel = topk_ids.numel()
    max_padded = numel + num_experts * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    dev = topk_ids.device
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    lib = load()
    nb = ctypes.c_size_t(0)
    check(lib.mstar_moe_align_scratch_size(numel, num_experts, ctypes.byref(nb)), "moe_align_block_size")
    scratch = torch.empty(max(nb.value, 4), dtype=torch.uint8, device=dev)
    check(lib.mstar_moe_align_block_size(
        ptr(topk_ids), dtype_code(topk_ids.dtype), numel, num_experts, block_size,
        ptr(sorted_ids), max_padded, ptr(expert_ids), max_blocks, ptr(ntpp), None, None,
        ptr(scratch), nb.value, stream_of(topk_ids)), "moe_align_block_size")
    return sorted_ids, expert_ids, ntpp


@moe_align_block_size.register_fake
def _(topk_ids, block_size, num_experts):
    max_padded = topk_ids.numel() + num_experts * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    return (topk_ids.new_empty(max_padded, dtype=torch.int32),
            topk_ids.new_empty(max_blocks, dtype=torch.int32),
            topk_ids.new_empty(1, dtype=torch.int32))


@torch.library.custom_op(f"{_NS}::moe_route", mutates_args=())
@_on_device
def moe_route(logits: torch.Tensor, top_k: int, renormalize: bool, block_size: int
              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Softmax top-k and alignment in one call: (weights fp32, ids int64,
    sorted_token_ids, expert_ids, num_tokens_post_padded)."""
    _lib.require_gpu(logits)
    logits = logits.contiguous()
    M, E = logits.shape
    numel = M * top_k
    max_padded = numel + E * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    dev = logits.device
    w = torch.empty(M, top_k, dtype=torch.float32, device=dev)
    ids = torch.empty(M, top_k, dtype=torch.int64, device=dev)
    sorted_ids = torch.empty(max_padded, dtype=torch.int32, device=dev)
    expert_ids = torch.empty(max_blocks, dtype=torch.int32, device=dev)
    ntpp = torch.empty(1, dtype=torch.int32, device=dev)
    lib = load()
    nb = ctypes.c_size_t(0)
    check(lib.mstar_moe_route_scratch_size(M, E, top_k, ctypes.byref(nb)), "moe_route")
    scratch = torch.empty(max(nb.value, 4), dtype=torch.uint8, device=dev)
    check(lib.mstar_moe_route(ptr(logits), dtype_code(logits.dtype), M, E, top_k, int(renormalize),
                              ptr(w), None, ptr(ids), block_size, ptr(sorted_ids), max_padded,
                              ptr(expert_ids), max_blocks, ptr(ntpp), None, None, ptr(scratch),
                              nb.value, stream_of(logits)), "moe_route")
    return w, ids, sorted_ids, expert_ids, ntpp


@moe_route.register_fake
def _(logits, top_k, renormalize, block_size):
    M, E = logits.shape
    max_padded = M * top_k + E * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    return (logits.new_empty(M, top_k, dtype=torch.float32),
            logits.new_empty(M, top_k, dtype=torch.int64),
            logits.new_empty(max_padded, dtype=torch.int32),
            logits.new_empty(max_blocks, dtype=torch.int32),
            logits.new_empty(1, dtype=torch.int32))


# --------------------------------------------------------------- elementwise
@torch.library.custom_op(f"{_NS}::act_and_mul", mutates_args=("out",))
@_on_device
def act_and_mul(gate_up: torch.Tensor, out: torch.Tensor, activation: int) -> None:
    _lib.require_gpu(gate_up, out)
    if not (gate_up.is_contiguous() and out.is_contiguous()):
        raise ValueError("act_and_mul: tensors must be contiguous")
    if gate_up.shape[0] != out.shape[0] or gate_up.shape[1] != 2 * out.shape[1]:
        raise ValueError("act_and_mul: expected gate_up [R, 2I] and out [R, I]")
    if gate_up.dtype != out.dtype:
        raise ValueError("act_and_mul: dtype mismatch")
    check(load().mstar_moe_act_and_mul(ptr(gate_up), ptr(out), dtype_code(out.dtype),
                                       out.shape[0], out.shape[1], activation, stream_of(out)),
          "act_and_mul")


@torch.library.custom_op(f"{_NS}::moe_sum_reduce", mutates_args=("output",))
@_on_device
def moe_sum_reduce(input: torch.Tensor, output: torch.Tensor, routed_scaling_factor: float) -> None:
    _lib.require_gpu(input, output)
    if not (input.is_contiguous() and output.is_contiguous()):
        raise ValueError("moe_sum_reduce: tensors must be contiguous")
    if input.dtype != output.dtype:
        raise ValueError(f"moe_sum_reduce: input {input.dtype} and output {output.dtype} dtypes differ")
    T, K, H = input.shape
    if output.shape[0] != T or output.shape[1] != H:
        raise ValueError("moe_sum_reduce: output must be [tokens, hidden]")
    check(load().mstar_moe_sum_reduce(ptr(input), ptr(output), dtype_code(input.dtype), T, K, H,
                                      float(routed_scaling_factor), stream_of(input)),
          "moe_sum_reduce")


# ------------------------------------------------------------ grouped GEMM
@torch.library.custom_op(f"{_NS}::grouped_gemm", mutates_args=("C",))
@_on_device
def grouped_gemm(A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
                 topk_weights: Optional[torch.Tensor], sorted_token_ids: torch.Tensor,
                 expert_ids: torch.Tensor, num_tokens_post_padded: torch.Tensor,
                 num_valid_tokens: int, top_k: int, mul_routed_weight: bool,
                 block_size: int) -> None:
    _lib.require_gpu(A, B, C)
    if not (A.is_contiguous() and B.is_contiguous() and C.is_contiguous()):
        raise ValueError("grouped_gemm: A, B and C must be contiguous")
    if A.dtype != B.dtype or A.dtype != C.dtype:
        raise ValueError("grouped_gemm: A, B and C must share a dtype")
    E, N, K = B.shape
    if A.shape[-1] != K or C.shape[-1] != N:
        raise ValueError(f"grouped_gemm: A [.., {A.shape[-1]}] / C [.., {C.shape[-1]}] do not match B {tuple(B.shape)}")
    tw_dt = dtype_code(topk_weights.dtype) if topk_weights is not None else 0
    check(load().mstar_moe_grouped_gemm(
        ptr(A), ptr(B), ptr(C), ptr(topk_weights), tw_dt, ptr(sorted_token_ids), ptr(expert_ids),
        ptr(num_tokens_post_padded), N, K, sorted_token_ids.shape[0], num_valid_tokens, top_k,
        int(mul_routed_weight), block_size, dtype_code(A.dtype), stream_of(A)), "grouped_gemm")


# ------------------------------------------------------------ fused experts
def _check_scale(name, s, dtype, shape):
    if s is None:
        raise ValueError(f"fused_experts: quantised weights need {name}")
    if s.dtype != dtype:
        raise ValueError(f"fused_experts: {name} must be {dtype}, got {s.dtype}")
    if tuple(s.shape) != tuple(shape):
        raise ValueError(f"fused_experts: {name} must have shape {tuple(shape)}, got {tuple(s.shape)}")
    if not s.is_contiguous():
        raise ValueError(f"fused_experts: {name} must be contiguous")


def _check_fused_args(hidden, w1, w2, topk_weights, topk_ids, quant, w1_scale, w2_scale):
    if hidden.dim() != 2:
        raise ValueError("fused_experts: hidden_states must be 2-D [tokens, hidden]")
    if topk_weights.shape != topk_ids.shape or topk_ids.dim() != 2:
        raise ValueError("fused_experts: topk_weights and topk_ids must both be [tokens, top_k]")
    if w1.dim() != 3 or w2.dim() != 3 or w1.shape[0] != w2.shape[0]:
        raise ValueError("fused_experts: w1 and w2 must be [E, ., .] with the same E")
    if not (w1.is_contiguous() and w2.is_contiguous()):
        raise ValueError("fused_experts: w1 and w2 must be contiguous")
    M, H = hidden.shape
    if topk_ids.shape[0] != M:
        raise ValueError(f"fused_experts: topk_ids has {topk_ids.shape[0]} rows for {M} tokens")
    if topk_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError(f"fused_experts: topk_ids must be int32 or int64, got {topk_ids.dtype}")
    E = w1.shape[0]
    if quant == _lib.QUANT_W4A16:
        two_i, hk = w1.shape[1], w1.shape[2] * 8
        _, w2h, inter = w2.shape[0], w2.shape[1], w2.shape[2] * 8
    else:
        two_i, hk = w1.shape[1], w1.shape[2]
        w2h, inter = w2.shape[1], w2.shape[2]
    if hk != H:
        raise ValueError(f"fused_experts: w1 last dim {hk} != hidden {H}")
    if w2h != H:
        raise ValueError(f"fused_experts: w2 dim[1] {w2h} != hidden {H}")
    if two_i != 2 * inter:
        raise ValueError(f"fused_experts: w1 dim[1] {two_i} != 2 * w2 inter {2 * inter}")
    if quant == _lib.QUANT_FP8_W8A8:
        # 128 x 128 weight blocks, fp32 (amax / 448)
        _check_scale("w1_scale", w1_scale, torch.float32, (E, -(-two_i // 128), H // 128))
        _check_scale("w2_scale", w2_scale, torch.float32, (E, H // 128, inter // 128))
    elif quant == _lib.QUANT_W4A16:
        # one bf16 scale per row and group of 128 along K
        _check_scale("w1_scale", w1_scale, torch.bfloat16, (E, two_i, H // 128))
        _check_scale("w2_scale", w2_scale, torch.bfloat16, (E, H, inter // 128))
    return M, H, E, inter


@torch.library.custom_op(f"{_NS}::fused_experts", mutates_args=())
@_on_device
def fused_experts_op(hidden: torch.Tensor, w1: torch.Tensor, w2: torch.Tensor,
                     topk_weights: torch.Tensor, topk_ids: torch.Tensor, activation: int,
                     reduce_results: bool, quant: int, w1_scale: Optional[torch.Tensor],
                     w2_scale: Optional[torch.Tensor]) -> torch.Tensor:
    _lib.require_gpu(hidden, w1, w2, topk_weights, topk_ids)
    hidden = hidden.contiguous()  # the kernels read rows of H elements
    M, H, E, inter = _check_fused_args(hidden, w1, w2, topk_weights, topk_ids, quant, w1_scale, w2_scale)
    top_k = topk_ids.shape[1]
    lib = load()
    act_dt = dtype_code(hidden.dtype)
    nbytes = ctypes.c_size_t(0)
    check(lib.mstar_fused_moe_workspace_size(M, H, E, inter, top_k, quant, act_dt,
                                             int(reduce_results), ctypes.byref(nbytes)),
          "fused_experts")
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=hidden.device)
    shape = (M, H) if reduce_results else (M, top_k, H)
    out = torch.empty(shape, dtype=hidden.dtype, device=hidden.device)
    tw = topk_weights.contiguous()
    ids = topk_ids.contiguous()
    check(lib.mstar_fused_moe(
        ptr(hidden), act_dt, M, H, ptr(w1), ptr(w2), E, inter, quant, ptr(w1_scale), ptr(w2_scale),
        ptr(tw), dtype_code(tw.dtype), ptr(ids), dtype_code(ids.dtype), top_k, activation,
        int(reduce_results), ptr(out), ptr(ws), nbytes.value, stream_of(hidden)), "fused_experts")
    return out


@fused_experts_op.register_fake
def _(hidden, w1, w2, topk_weights, topk_ids, activation, reduce_results, quant, w1_scale, w2_scale):
    M, H = hidden.shape
    if reduce_results:
        return hidden.new_empty(M, H)
    return hidden.new_empty(M, topk_ids.shape[1], H)


@torch.library.custom_op(f"{_NS}::moe_layer", mutates_args=())
@_on_device
def moe_layer(hidden: torch.Tensor, router_logits: torch.Tensor, w1: torch.Tensor,
              w2: torch.Tensor, top_k: int, renormalize: bool, activation: int, quant: int,
              w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor]
              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Routed MoE layer from router logits: (out, topk_weights fp32, topk_ids int64)."""
    _lib.require_gpu(hidden, router_logits, w1, w2)
    hidden = hidden.contiguous()
    dummy_ids = torch.empty(hidden.shape[0], top_k, dtype=torch.int64, device=hidden.device)
    dummy_w = torch.empty(hidden.shape[0], top_k, dtype=torch.float32, device=hidden.device)
    M, H, E, inter = _check_fused_args(hidden, w1, w2, dummy_w, dummy_ids, quant, w1_scale, w2_scale)
    logits = router_logits.contiguous()
    if logits.shape != (M, E):
        raise ValueError(f"moe_layer: router_logits must be [{M}, {E}]")
    lib = load()
    act_dt = dtype_code(hidden.dtype)
    nbytes = ctypes.c_size_t(0)
    check(lib.mstar_moe_layer_workspace_size(M, H, E, inter, top_k, quant, act_dt,
                                             ctypes.byref(nbytes)), "moe_layer")
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=hidden.device)
    out = torch.empty(M, H, dtype=hidden.dtype, device=hidden.device)
    if _wait_checks_on() and torch.cuda.current_device() not in _WAIT_FAILURES:
        torch.cuda.synchronize()  # the counter before this process's first checked call
        _WAIT_FAILURES[torch.cuda.current_device()] = _layer_wait_failures()
    check(lib.mstar_moe_layer(
        ptr(hidden), act_dt, M, H, ptr(logits), dtype_code(logits.dtype), int(renormalize), ptr(w1),
        ptr(w2), E, inter, quant, ptr(w1_scale), ptr(w2_scale), top_k, activation, ptr(out),
        ptr(dummy_w), ptr(dummy_ids), ptr(ws), nbytes.value, stream_of(hidden)), "moe_layer")
    _check_layer_waits("moe_layer")
    return out, dummy_w, dummy_ids


@moe_layer.register_fake
def _(hidden, router_logits, w1, w2, top_k, renormalize, activation, quant, w1_scale, w2_scale):
    M, H = hidden.shape
    return (hidden.new_empty(M, H), hidden.new_empty(M, top_k, dtype=torch.float32),
            hidden.new_empty(M, top_k, dtype=torch.int64))


@torch.library.custom_op(f"{_NS}::moe_block", mutates_args=())
@_on_device
def moe_block(hidden: torch.Tensor, gate_weight: torch.Tensor, w1: torch.Tensor,
              w2: torch.Tensor, top_k: int, renormalize: bool, activation: int, quant: int,
              w1_scale: Optional[torch.Tensor], w2_scale: Optional[torch.Tensor]
              ) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Routed MoE layer from the hidden states (fused router + experts, one
    library call): (out, topk_weights fp32, topk_ids int64)."""
    _lib.require_gpu(hidden, gate_weight, w1, w2)
    hidden = hidden.contiguous()
    if hidden.dtype != torch.bfloat16 or gate_weight.dtype != torch.bfloat16:
        raise ValueError("moe_block: hidden states and gate weight must be bfloat16")
    dummy_ids = torch.empty(hidden.shape[0], top_k, dtype=torch.int64, device=hidden.device)
    dummy_w = torch.empty(hidden.shape[0], top_k, dtype=torch.float32, device=hidden.device)
    M, H, E, inter = _check_fused_args(hidden, w1, w2, dummy_w, dummy_ids, quant, w1_scale, w2_scale)
    gate_weight = gate_weight.contiguous()
    if tuple(gate_weight.shape) != (E, H):
        raise ValueError(f"moe_block: gate weight must be [{E}, {H}], got {tuple(gate_weight.shape)}")
    lib = load()
    act_dt = dtype_code(hidden.dtype)
    nbytes = ctypes.c_size_t(0)
    check(lib.mstar_moe_layer_workspace_size(M, H, E, inter, top_k, quant, act_dt,
                                             ctypes.byref(nbytes)), "moe_block")
    ws = torch.empty(max(nbytes.value, 1), dtype=torch.uint8, device=hidden.device)
    out = torch.empty(M, H, dtype=hidden.dtype, device=hidden.device)
    check(lib.mstar_moe_block(
        ptr(hidden), act_dt, M, H, ptr(gate_weight), int(renormalize), ptr(w1), ptr(w2), E, inter,
        quant, ptr(w1_scale), ptr(w2_scale), top_k, activation, ptr(out), ptr(dummy_w),
        ptr(dummy_ids), None, ptr(ws), nbytes.value, stream_of(hidden)), "moe_block")
    return out, dummy_w, dummy_ids


@moe_block.register_fake
def _(hidden, gate_weight, w1, w2, top_k, renormalize, activation, quant, w1_scale, w2_scale):
    M, H = hidden.shape
    return (hidden.new_empty(M, H), hidden.new_empty(M, top_k, dtype=torch.float32),
            hidden.new_empty(M, top_k, dtype=torch.int64))


# ---------------------------------------------------------- FP8 quant / GEMM
@torch.library.custom_op(f"{_NS}::quant_fp8_per_token_group", mutates_args=())
@_on_device
def quant_fp8_per_token_group(x: torch.Tensor, group_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    _lib.require_gpu(x)
    x = x.contiguous()
    R, C = x.shape
    q = torch.empty(R, C, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(R, C // group_size, dtype=torch.float32, device=x.device)
    check(load().mstar_quant_fp8_per_token_group(ptr(x), dtype_code(x.dtype), R, C, group_size,
                                                 ptr(q), ptr(s), stream_of(x)),
          "quant_fp8_per_token_group")
    return q, s


@quant_fp8_per_token_group.register_fake
def _(x, group_size):
    R, C = x.shape
    return x.new_empty(R, C, dtype=torch.float8_e4m3fn), x.new_empty(R, C // group_size, dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::quant_fp8_per_token", mutates_args=())
@_on_device
def quant_fp8_per_token(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    _lib.require_gpu(x)
    x = x.contiguous()
    R, C = x.shape
    q = torch.empty(R, C, dtype=torch.float8_e4m3fn, device=x.device)
    s = torch.empty(R, dtype=torch.float32, device=x.device)
    check(load().mstar_quant_fp8_per_token(ptr(x), dtype_code(x.dtype), R, C, ptr(q), ptr(s),
                                           stream_of(x)), "quant_fp8_per_token")
    return q, s


@quant_fp8_per_token.register_fake
def _(x):
    R, C = x.shape
    return x.new_empty(R, C, dtype=torch.float8_e4m3fn), x.new_empty(R, dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::fp8_scaled_mm", mutates_args=())
@_on_device
def fp8_scaled_mm(a: torch.Tensor, a_scale: torch.Tensor, w: torch.Tensor,
                  w_scale: torch.Tensor) -> torch.Tensor:
    _lib.require_gpu(a, a_scale, w, w_scale)
    M, K = a.shape
    N, K2 = w.shape
    if K != K2:
        raise ValueError(f"fp8_scaled_mm: K mismatch {K} vs {K2}")
    if a.dtype != torch.float8_e4m3fn or w.dtype != torch.float8_e4m3fn:
        raise ValueError("fp8_scaled_mm: operands must be float8_e4m3fn")
    a, a_scale, w, w_scale = a.contiguous(), a_scale.contiguous(), w.contiguous(), w_scale.contiguous()
    out = torch.empty(M, N, dtype=torch.bfloat16, device=a.device)
    check(load().mstar_fp8_scaled_mm(ptr(a), ptr(a_scale), ptr(w), ptr(w_scale), ptr(out), M, N, K,
                                     stream_of(a)), "fp8_scaled_mm")
    return out


@fp8_scaled_mm.register_fake
def _(a, a_scale, w, w_scale):
    return a.new_empty(a.shape[0], w.shape[0], dtype=torch.bfloat16)
