"""Shared helpers for the parity tests."""
from __future__ import annotations

import torch

# Tolerance stated for floating-point outputs: max |out - ref| <= 2e-2 * max|ref|
# and mean |out - ref| <= 1e-3 * rms(ref).
MAX_REL = 2e-2
MEAN_ABS_OF_RMS = 1e-3


def moe_errors(out: torch.Tensor, ref: torch.Tensor):
    o = out.detach().float().cpu()
    r = ref.detach().float().cpu()
    err = (o - r).abs()
    scale = r.abs().max().clamp_min(1e-30)
    rms = r.pow(2).mean().sqrt().clamp_min(1e-30)
    return float(err.max() / scale), float(err.mean() / rms)


# (what, max_rel, mean_abs/rms) of every comparison, written out by conftest.
RECORDS: list = []


def assert_moe_close(out: torch.Tensor, ref: torch.Tensor, max_rel=MAX_REL,
                     mean_of_rms=MEAN_ABS_OF_RMS, what=""):
    assert out.shape == ref.shape, (out.shape, ref.shape)
    assert torch.isfinite(out.float()).all(), f"{what}: non-finite output"
    mr, ma = moe_errors(out, ref)
    RECORDS.append({"what": what, "max_rel": mr, "mean_abs_over_rms": ma})
    assert mr <= max_rel and ma <= mean_of_rms, (
        f"{what}: max_rel={mr:.3e} (<= {max_rel}), mean_abs/rms={ma:.3e} (<= {mean_of_rms})")


def align_brute_force(ids, block_size: int, num_experts: int):
    """Pure-Python statement of the moe_align_block_size contract
    (mstar/utils/fused_moe/align.py:55-103, csrc/moe_align_block_size.cu:207-271):
    walk experts in order, list each expert's slots in ascending order, pad
    each expert's run to a multiple of block_size with `numel`, fill the
    rest of the buffer with `numel`, and give every block its expert."""
    flat = [int(v) for v in ids.reshape(-1).tolist()]
    numel = len(flat)
    max_padded = numel + num_experts * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    sorted_ids = []
    expert_ids = []
    for e in range(num_experts):
        run = [i for i, v in enumerate(flat) if v == e]
        if not run:
            continue
        while len(run) % block_size:
            run.append(numel)
        expert_ids += [e] * (len(run) // block_size)
        sorted_ids += run
    ntpp = len(sorted_ids)
    sorted_ids += [numel] * (max_padded - ntpp)
    expert_ids += [0] * (max_blocks - len(expert_ids))
    return sorted_ids, expert_ids, ntpp
