"""MoE blocks and the router (drop-in for mstar/model/components/moe.py).

* :class:`TopKRouter` -- gate projection, softmax, top-k and renormalisation
  (moe.py:85-140): one fused HIP launch for bf16 states and weights (the
  reference's dtype), else ``F.linear`` then the HIP softmax-top-k kernel;
  returns ``(weights fp32, ids int64, None)`` like the reference's 3-tuple
  router contract.
* :func:`dispatch` -- the fused path (moe.py:188-205 minus the naive
  fallback: these kernels are the only compute path; CPU tensors raise).
* :class:`SparseMoeBlock` / :class:`SparseMoeBlockWithSharedExpert` --
  the reference blocks (moe.py:208-328) with the same parameter layout
  (``experts.gate_up_proj [E, 2I, H]`` rows ``[gate; up]``,
  ``experts.down_proj [E, H, I]``) plus :meth:`quantize` to switch the
  experts to FP8 (block 128x128) or W4A16 (group 128) storage.
* :class:`ParallelSparseMoeBlock` / :class:`ParallelSparseMoeBlockWithSharedExpert`
  -- the tensor-parallel blocks (moe.py:378-591): experts sharded along the
  intermediate size, per-expert weight loaders, the routed output summed
  over the group (RCCL through ``torch.distributed``).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import nn

from . import ops, quant
from .fused_moe import fused_experts


class TopKRouter(nn.Module):
    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 norm_topk_prob: bool = True) -> None:
        super().__init__()
        self.top_k = num_experts_per_tok
        self.num_experts = num_experts
        self.norm_topk_prob = norm_topk_prob
        self.weight = nn.Parameter(torch.zeros(num_experts, hidden_size))

    def fused_ok(self, hidden_states: torch.Tensor) -> bool:
        """Whether the fused router kernel takes these states (bf16 states
        and weight, at most 256 experts, hidden size a multiple of 32)."""
        return (hidden_states.dtype == torch.bfloat16 and self.weight.dtype == torch.bfloat16
                and self.num_experts <= 256 and hidden_states.shape[-1] % 32 == 0)

    def forward(self, hidden_states: torch.Tensor, router_states: torch.Tensor | None = None):
        hidden_states = hidden_states.reshape(-1, hidden_states.shape[-1])
        if self.fused_ok(hidden_states):
            w, ids = ops.router(hidden_states, self.weight, self.top_k, self.norm_topk_prob)
            return w, ids, None
        router_logits = F.linear(hidden_states, self.weight)
        w, ids = ops.topk_softmax(router_logits, self.top_k, self.norm_topk_prob)
        return w, ids, None


class _Experts(nn.Module):
    def __init__(self, num_experts: int, hidden_size: int, inter: int) -> None:
        super().__init__()
        self.gate_up_proj = nn.Parameter(torch.empty(num_experts, 2 * inter, hidden_size))
        self.down_proj = nn.Parameter(torch.empty(num_experts, hidden_size, inter))
        self.quant: str | None = None
        self.register_buffer("w1_scale", None)
        self.register_buffer("w2_scale", None)

    @torch.no_grad()
    def quantize(self, mode: str) -> None:
        """Replace the bf16 expert weights by ``mode`` storage in place."""
        if self.quant is not None:
            raise RuntimeError(f"experts already quantised ({self.quant})")
        w1, w2 = self.gate_up_proj.data, self.down_proj.data
        if mode == "fp8_w8a8":
            q1, s1 = quant.quantize_fp8_block(w1)
            q2, s2 = quant.quantize_fp8_block(w2)
        elif mode == "w4a16":
            q1, s1 = quant.quantize_int4_group(w1)
            q2, s2 = quant.quantize_int4_group(w2)
        else:
            raise ValueError(f"unknown quantisation mode {mode!r}")
        self.gate_up_proj = nn.Parameter(q1, requires_grad=False)
        self.down_proj = nn.Parameter(q2, requires_grad=False)
        self.w1_scale = s1
        self.w2_scale = s2
        self.quant = mode


def _quant_code(mode: str | None) -> int:
    from ._lib import QUANT_FP8_W8A8, QUANT_NONE, QUANT_W4A16
    return {None: QUANT_NONE, "fp8_w8a8": QUANT_FP8_W8A8, "w4a16": QUANT_W4A16}[mode]


def dispatch(hidden_states, experts: _Experts, num_experts, selected_experts, routing_weights):
    return fused_experts(hidden_states, experts.gate_up_proj, experts.down_proj, routing_weights,
                         selected_experts, quant=experts.quant, w1_scale=experts.w1_scale,
                         w2_scale=experts.w2_scale)


class SparseMoeBlock(nn.Module):
    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 moe_intermediate_size: int, norm_topk_prob: bool = True,
                 router: nn.Module | None = None) -> None:
        super().__init__()
        self.hidden_size = hidden_size
        self.num_experts = num_experts
        self.num_experts_per_tok = num_experts_per_tok
        self.moe_intermediate_size = moe_intermediate_size
        self.gate = router if router is not None else TopKRouter(
            hidden_size, num_experts, num_experts_per_tok, norm_topk_prob)
        self.experts = _Experts(num_experts, hidden_size, moe_intermediate_size)

    def quantize(self, mode: str) -> "SparseMoeBlock":
        self.experts.quantize(mode)
        return self

    def routed(self, flat, router_states=None):
        """Routed experts of ``flat [T, H]`` -> ``(out, router_states_next)``.
        With the default router the whole routed layer -- gate projection,
        softmax top-k, align, both GEMMs, the top-k sum -- is one library
        call (the fused router for bf16 states, as TopKRouter uses it; for
        other dtypes the gate projection is an ``F.linear`` first)."""
        if type(self.gate) is TopKRouter:
            ex = self.experts
            if self.gate.fused_ok(flat):
                out, _, _ = ops.moe_block(flat, self.gate.weight, ex.gate_up_proj, ex.down_proj,
                                          self.gate.top_k, self.gate.norm_topk_prob, 0,
                                          _quant_code(ex.quant), ex.w1_scale, ex.w2_scale)
                return out, None
            logits = F.linear(flat, self.gate.weight)
            out, _, _ = ops.moe_layer(flat, logits, ex.gate_up_proj, ex.down_proj, self.gate.top_k,
                                      self.gate.norm_topk_prob, 0, _quant_code(ex.quant),
                                      ex.w1_scale, ex.w2_scale)
            return out, None
        w, ids, router_states_next = self.gate(flat, router_states)
        return dispatch(flat, self.experts, self.num_experts, ids, w), router_states_next

    def forward(self, hidden_states, router_states=None, *, return_router_states: bool = False):
        input_shape = hidden_states.shape
        flat = hidden_states.view(-1, hidden_states.shape[-1]).contiguous()
        out, router_states_next = self.routed(flat, router_states)
        out = out.view(input_shape)
        return (out, router_states_next) if return_router_states else out


class SparseMoeBlockWithSharedExpert(SparseMoeBlock):
    """``out = routed(x) + sigmoid(shared_gate(x)) * shared_expert(x)`` (moe.py:264-328)."""

    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 moe_intermediate_size: int, shared_expert: nn.Module,
                 norm_topk_prob: bool = False, router: nn.Module | None = None) -> None:
        super().__init__(hidden_size, num_experts, num_experts_per_tok, moe_intermediate_size,
                         norm_topk_prob, router)
        self.shared_expert = shared_expert
        self.shared_expert_gate = nn.Linear(hidden_size, 1, bias=False)

    def forward(self, hidden_states, router_states=None, *, return_router_states: bool = False):
        input_shape = hidden_states.shape
        flat = hidden_states.view(-1, hidden_states.shape[-1]).contiguous()
        shared = self.shared_expert(flat)
        routed, router_states_next = self.routed(flat, router_states)
        out = (routed + torch.sigmoid(self.shared_expert_gate(flat)) * shared).view(input_shape)
        return (out, router_states_next) if return_router_states else out


# ---------------------------------------------------------------------------
# Tensor-parallel blocks (moe.py:378-591): experts sharded along the
# intermediate dimension, the routed output summed over the group.
# ---------------------------------------------------------------------------
class ProcessGroupComm:
    """The communication-group interface the blocks use (``rank``,
    ``world_size``, in-place sum ``all_reduce``; the reference's
    ``CommGroup``, mstar/distributed/communication.py:8-36, fits it as is)
    over a ``torch.distributed`` group.  On ROCm the ``nccl`` backend is
    RCCL and reduces device tensors directly; a ``gloo`` group is handed a
    synchronous host copy (gloo collectives take CPU tensors)."""

    def __init__(self, group=None) -> None:
        import torch.distributed as dist
        self.group = group
        self.rank = dist.get_rank(group)
        self.world_size = dist.get_world_size(group)

    @classmethod
    def trivial(cls) -> "ProcessGroupComm":
        c = cls.__new__(cls)
        c.group, c.rank, c.world_size = None, 0, 1
        return c

    def all_reduce(self, t: torch.Tensor) -> torch.Tensor:
        if self.world_size == 1:
            return t
        import torch.distributed as dist
        if t.is_cuda and dist.get_backend(self.group) == "gloo":
            h = t.cpu()
            dist.all_reduce(h, group=self.group)
            t.copy_(h)
        else:
            dist.all_reduce(t, group=self.group)
        return t


def _divide(n: int, d: int) -> int:
    if n % d:
        raise ValueError(f"{n} is not divisible by {d}")
    return n // d


@torch.no_grad()
def gate_up_weight_loader(tp_rank: int, tp_size: int, full_inter: int, param: nn.Parameter,
                          loaded_weight: torch.Tensor, loaded_shard_id: str) -> None:
    """One expert's ``gate_proj`` / ``up_proj`` ``[inter, hidden]``
    (``loaded_shard_id`` ``"gate:N"`` / ``"up:N"``) into rank ``tp_rank``'s
    ``gate_up_proj [E, 2 I/P, H]``: its row slice, gate rows first
    (moe.py:335-359)."""
    kind, expert = loaded_shard_id.split(":")
    shard = _divide(full_inter, tp_size)
    rows = loaded_weight[tp_rank * shard:(tp_rank + 1) * shard, :]
    if kind not in ("gate", "up"):
        raise ValueError(f"unknown shard id {loaded_shard_id!r}")
    off = 0 if kind == "gate" else shard
    param.data[int(expert), off:off + shard, :] = rows


@torch.no_grad()
def down_proj_weight_loader(tp_rank: int, tp_size: int, full_inter: int, param: nn.Parameter,
                            loaded_weight: torch.Tensor, loaded_shard_id: str) -> None:
    """One expert's ``down_proj`` ``[hidden, inter]`` (``"down:N"``) into
    rank ``tp_rank``'s ``down_proj [E, H, I/P]``: its column slice
    (moe.py:362-375)."""
    shard = _divide(full_inter, tp_size)
    param.data[int(loaded_shard_id.split(":")[1])] = loaded_weight[:, tp_rank * shard:(tp_rank + 1) * shard]


class _TensorParallel:
    """Shared by the two tensor-parallel blocks: the rank's expert shard, its
    weight loaders, and the group sum of the routed output."""

    def _init_tp(self, comm_group, full_inter: int) -> int:
        self.comm_group = comm_group if comm_group is not None else ProcessGroupComm.trivial()
        return _divide(full_inter, self.comm_group.world_size)

    def _attach_weight_loaders(self) -> None:
        from functools import partial
        r, p, full = self.comm_group.rank, self.comm_group.world_size, self.moe_intermediate_size
        self.experts.gate_up_proj.weight_loader = partial(gate_up_weight_loader, r, p, full)
        self.experts.down_proj.weight_loader = partial(down_proj_weight_loader, r, p, full)

    def _apply(self, fn, recurse=True):
        result = super()._apply(fn, recurse=recurse)
        if hasattr(self, "comm_group"):
            self._attach_weight_loaders()
        return result

    def routed(self, flat, router_states=None):
        """The rank's partial routed output (its shard of every expert,
        top-k sum included), then the sum over the group.  The reference
        (``_dispatch_tp``, moe.py:467-482) sums the top-k in fp32 and
        stores bf16 before its all-reduce; the fused layer does the same."""
        out, router_states_next = super().routed(flat, router_states)
        self.comm_group.all_reduce(out)
        return out, router_states_next


class ParallelSparseMoeBlock(_TensorParallel, SparseMoeBlock):
    """Tensor-parallel ``SparseMoeBlock`` (moe.py:378-482).  With a one-rank
    group the forward is ``SparseMoeBlock``'s."""

    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 moe_intermediate_size: int, norm_topk_prob: bool = True,
                 router: nn.Module | None = None, comm_group=None) -> None:
        SparseMoeBlock.__init__(self, hidden_size, num_experts, num_experts_per_tok,
                                moe_intermediate_size, norm_topk_prob, router)
        shard = self._init_tp(comm_group, moe_intermediate_size)
        self.experts = _Experts(num_experts, hidden_size, shard)
        self._attach_weight_loaders()


class ParallelSparseMoeBlockWithSharedExpert(_TensorParallel, SparseMoeBlockWithSharedExpert):
    """Tensor-parallel ``SparseMoeBlockWithSharedExpert`` (moe.py:485-591).
    The shared expert handles its own reduction (a row-parallel MLP built on
    the same group, as in the reference)."""

    def __init__(self, hidden_size: int, num_experts: int, num_experts_per_tok: int,
                 moe_intermediate_size: int, shared_expert: nn.Module,
                 norm_topk_prob: bool = False, router: nn.Module | None = None,
                 comm_group=None) -> None:
        SparseMoeBlockWithSharedExpert.__init__(self, hidden_size, num_experts, num_experts_per_tok,
                                                moe_intermediate_size, shared_expert,
                                                norm_topk_prob, router)
        shard = self._init_tp(comm_group, moe_intermediate_size)
        self.experts = _Experts(num_experts, hidden_size, shard)
        self._attach_weight_loaders()
