"""FP8 expert weights at load time and on disk.

The reference stacks each expert's ``gate_proj`` / ``up_proj`` / ``down_proj``
into the fused ``gate_up_proj [E, 2I/P, H]`` and ``down_proj [E, H, I/P]``
parameters while a checkpoint loads, taking tensor-parallel rank ``r``'s
slice of the intermediate dimension (``_gate_up_weight_loader`` and
``_down_proj_weight_loader``, mstar/model/components/moe.py:335-375).  The
loaders here do the same slicing and store the slice directly as FP8 with
128x128 block scales (``quant.quantize_fp8_block``: scale = amax/448), so a
bf16 checkpoint is quantised expert by expert without materialising the
bf16 stack.  Blocks are local to the slice (``I/P`` must be a multiple of
128), so the result equals quantising the stacked bf16 parameter.

On disk the quantised experts are one safetensors file:

* ``experts.gate_up_proj.qweight`` e4m3fn ``[E, 2I/P, H]`` (rows ``[gate; up]``)
* ``experts.gate_up_proj.scale``   fp32   ``[E, 2I/(128P), H/128]``
* ``experts.down_proj.qweight``    e4m3fn ``[E, H, I/P]``
* ``experts.down_proj.scale``      fp32   ``[E, H/128, I/(128P)]``

with metadata ``format = mstar-amd-fp8-block``, ``block = 128,128``.
"""
from __future__ import annotations

import torch

from . import quant

BLOCK = 128
FORMAT = "mstar-amd-fp8-block"
_KEYS = ("experts.gate_up_proj.qweight", "experts.gate_up_proj.scale",
         "experts.down_proj.qweight", "experts.down_proj.scale")


def _shard(full_inter: int, tp_size: int) -> int:
    if full_inter % tp_size != 0:
        raise ValueError(f"{full_inter} is not divisible by {tp_size}")
    shard = full_inter // tp_size
    if shard % BLOCK != 0:
        raise ValueError(f"FP8 block loading needs the per-rank intermediate size ({shard}) "
                         f"to be a multiple of {BLOCK}")
    return shard


def empty_fp8_experts(num_experts: int, hidden: int, full_inter: int, tp_size: int = 1,
                      device: torch.device | str | None = None):
    """Allocate ``(w1_q, w1_s, w2_q, w2_s)`` for one rank's slice."""
    if hidden % BLOCK != 0:
        raise ValueError(f"hidden size {hidden} is not a multiple of {BLOCK}")
    shard = _shard(full_inter, tp_size)
    f8 = torch.float8_e4m3fn
    return (torch.empty(num_experts, 2 * shard, hidden, dtype=f8, device=device),
            torch.empty(num_experts, 2 * shard // BLOCK, hidden // BLOCK, dtype=torch.float32, device=device),
            torch.empty(num_experts, hidden, shard, dtype=f8, device=device),
            torch.empty(num_experts, hidden // BLOCK, shard // BLOCK, dtype=torch.float32, device=device))


@torch.no_grad()
def fp8_gate_up_weight_loader(tp_rank: int, tp_size: int, full_inter: int, w1_q: torch.Tensor,
                              w1_s: torch.Tensor, loaded_weight: torch.Tensor,
                              loaded_shard_id: str) -> None:
    """One expert's ``gate_proj`` or ``up_proj`` (``[inter, hidden]``,
    ``loaded_shard_id`` = ``"gate:N"`` / ``"up:N"``) into rank ``tp_rank``'s
    FP8 ``gate_up_proj``: gate rows first, then up rows (moe.py:335-359)."""
    kind, expert = loaded_shard_id.split(":")
    e = int(expert)
    shard = _shard(full_inter, tp_size)
    start = tp_rank * shard
    q, s = quant.quantize_fp8_block(loaded_weight[start:start + shard, :].to(w1_s.device))
    if kind == "gate":
        row0 = 0
    elif kind == "up":
        row0 = shard
    else:
        raise ValueError(f"unknown shard id {loaded_shard_id!r}")
    w1_q[e, row0:row0 + shard, :] = q
    w1_s[e, row0 // BLOCK:(row0 + shard) // BLOCK, :] = s


@torch.no_grad()
def fp8_down_proj_weight_loader(tp_rank: int, tp_size: int, full_inter: int, w2_q: torch.Tensor,
                                w2_s: torch.Tensor, loaded_weight: torch.Tensor,
                                loaded_shard_id: str) -> None:
    """One expert's ``down_proj`` (``[hidden, inter]``, ``"down:N"``) into
    rank ``tp_rank``'s FP8 ``down_proj``: its column slice (moe.py:362-375)."""
    e = int(loaded_shard_id.split(":")[1])
    shard = _shard(full_inter, tp_size)
    start = tp_rank * shard
    q, s = quant.quantize_fp8_block(loaded_weight[:, start:start + shard].to(w2_s.device))
    w2_q[e] = q
    w2_s[e] = s


def save_fp8_experts(path: str, w1_q: torch.Tensor, w1_s: torch.Tensor, w2_q: torch.Tensor,
                     w2_s: torch.Tensor) -> None:
    """Write one rank's FP8 experts in the block-scaled safetensors format."""
    from safetensors.torch import save_file
    tensors = dict(zip(_KEYS, (w1_q, w1_s, w2_q, w2_s)))
    save_file({k: v.detach().contiguous().cpu() for k, v in tensors.items()}, path,
              metadata={"format": FORMAT, "block": f"{BLOCK},{BLOCK}", "scale": "amax/448"})


def load_fp8_experts(path: str, device: torch.device | str | None = None):
    """Read ``(w1_q, w1_s, w2_q, w2_s)`` written by :func:`save_fp8_experts`
    (safetensors: no code in the file is executed)."""
    from safetensors import safe_open
    with safe_open(path, framework="pt", device="cpu") as f:
        meta = f.metadata() or {}
        if meta.get("format") != FORMAT or meta.get("block") != f"{BLOCK},{BLOCK}":
            raise ValueError(f"{path}: not a {FORMAT} file (metadata {meta})")
        out = tuple(f.get_tensor(k) for k in _KEYS)
    if out[0].dtype != torch.float8_e4m3fn or out[2].dtype != torch.float8_e4m3fn:
        raise ValueError(f"{path}: expert weights are not e4m3fn")
    return tuple(t.to(device) for t in out) if device is not None else out
