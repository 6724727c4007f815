"""Capture integration: the MoE block traced by torch.compile (dynamic=False,
fullgraph -- the library ops have fake implementations, so nothing breaks
the graph) and captured in a HIP graph, as the reference's
CudaGraphRunner does at its decode / prefill buckets
(mstar/engine/cuda_graph_runner.py:599-640).  Every replay, with eager work in
between, must equal the eager result bit for bit."""
from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _block(seed=0):
    from mstar_amd.moe import SparseMoeBlock
    H, E, k, I = 2048, 128, 8, 768
    g = torch.Generator().manual_seed(seed)
    b = SparseMoeBlock(H, E, k, I)
    with torch.no_grad():
        b.gate.weight.copy_(torch.randn(E, H, generator=g) * 0.02)
        b.experts.gate_up_proj.copy_(torch.randn(E, 2 * I, H, generator=g) * 0.02)
        b.experts.down_proj.copy_(torch.randn(E, H, I, generator=g) * 0.02)
    return b.to(DEV).to(torch.bfloat16).quantize("fp8_w8a8")


@pytest.mark.parametrize("M", [32, 512])
def test_compiled_block_under_hip_graph(M):
    torch._dynamo.reset()
    block = _block()
    x = torch.randn(M, 2048, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        eager = block(x)
        compiled = torch.compile(block, backend="aot_eager", dynamic=False, fullgraph=True)
        assert torch.equal(compiled(x), eager)
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            compiled(x)
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = compiled(x)
        for _ in range(3):
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
            _ = block(x)  # eager work between replays
            torch.cuda.synchronize()
