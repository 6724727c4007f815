"""Write the seeded golden fixtures under tests/golden/ (run from the repo root:
``python -m tests.golden.make_golden``).

The reference ships no fixtures for this path and is not executed here; the
fixtures are the oracle's outputs on the BASELINE.json inputs (seed 0),
stored so the GPU tests compare against fixed vectors and the CPU suite can
detect oracle drift.  Only small arrays are stored: routing ids/weights,
alignment outputs, and the tiny config's full MoE output (its inputs are
regenerated from the seed).
"""
from __future__ import annotations

import os

import numpy as np
import torch

from oracle import moe_oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))

# name -> (M, E, top_k, bias, block_size, renormalize)
ROUTE_CASES = {
    "route_tiny": (64, 8, 2, False, 64, True),        # config 1 (M > E -> BM 64)
    "route_decode": (32, 128, 8, False, 16, True),    # config 2 (M <= E -> BM 16)
    "route_prefill512": (512, 128, 8, True, 64, True),  # config 3, M=512 of the sweep
}


def route_logits(M: int, E: int, bias: bool) -> torch.Tensor:
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(M, E, generator=g)
    return logits + O.zipf_bias(E) if bias else logits


def compute(name: str) -> dict[str, np.ndarray]:
    if name in ROUTE_CASES:
        M, E, k, bias, bm, renorm = ROUTE_CASES[name]
        logits = route_logits(M, E, bias)
        w, ids = O.router_topk_softmax(logits, k, renorm)
        s, e, n = O.moe_align_block_size(ids.numpy(), bm, E)
        return {"logits": logits.numpy(), "topk_weights": w.numpy(), "topk_ids": ids.numpy(),
                "sorted_token_ids": s, "expert_ids": e, "num_tokens_post_padded": n}
    if name == "moe_tiny_bf16":
        x, w1, w2, logits = O.make_moe_inputs(64, 256, 8, 2, 512, seed=0)
        w, ids = O.router_topk_softmax(logits, 2, True)
        out = O.fused_experts_rounding(x, w1, w2, w, ids)
        naive = O.naive_dispatch(x, w1, w2, 8, ids, w)
        return {"topk_ids": ids.numpy(), "out_bits": out.view(torch.int16).numpy(),
                "naive_bits": naive.view(torch.int16).numpy()}
    raise KeyError(name)


NAMES = list(ROUTE_CASES) + ["moe_tiny_bf16"]


def main() -> None:
    for name in NAMES:
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **compute(name))
        print("wrote", name)


if __name__ == "__main__":
    main()
