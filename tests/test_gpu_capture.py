"""Capture integration: the MoE block traced by torch.compile (dynamic=False,
fullgraph -- the library ops have fake implementations, so nothing breaks
the graph) and captured in a HIP graph, as the reference's
CudaGraphRunner does at its decode / prefill buckets
(mstar/engine/cuda_graph_runner.py:599-640): first through aot_eager, then
through inductor with the reference's own mode
(``max-autotune-no-cudagraphs``, cuda_graph_runner.py:617-620) at decode
buckets 1, 8, 32 and prefill buckets 128, 2048 (submodules.py:709-720).
The library ops must reach the inductor output as opaque extern calls, and
every replay, with eager work in between, must equal the eager result bit
for bit."""
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


def _capture_and_check(fn, x, eager, replays=3):
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn(x)
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = fn(x)
    for _ in range(replays):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        _ = fn(x)  # eager work between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("M", [1, 8, 32, 128, 2048])
def test_inductor_block_under_hip_graph(M):
    from torch._inductor.utils import run_and_get_code
    torch._dynamo.reset()
    block = _block()
    x = torch.randn(M, 2048, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).to(DEV)
    print(f"inductor max-autotune-no-cudagraphs M={M}", flush=True)
    with torch.no_grad():
        eager = block(x)
        compiled = torch.compile(block, mode="max-autotune-no-cudagraphs", dynamic=False,
                                 fullgraph=True)
        out, code = run_and_get_code(compiled, x)
        src = "\n".join(code)
        assert "torch.ops.mstar_moe.moe_block" in src, src[-3000:]
        assert torch.equal(out, eager)
        _capture_and_check(compiled, x, eager)


def test_inductor_shared_expert_block():
    """The talker's block: the routed call stays opaque while inductor
    generates the shared expert's gate and combine around it."""
    from torch._inductor.utils import run_and_get_code
    from mstar_amd.moe import SparseMoeBlockWithSharedExpert
    torch._dynamo.reset()
    H, E, k, I = 1024, 128, 8, 384
    g = torch.Generator().manual_seed(9)
    shared = torch.nn.Linear(H, H, bias=False)
    b = SparseMoeBlockWithSharedExpert(H, E, k, I, shared_expert=shared)
    with torch.no_grad():
        for p in b.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.02)
    b = b.to(DEV).to(torch.bfloat16).quantize("fp8_w8a8")
    x = torch.randn(32, H, generator=g).to(torch.bfloat16).to(DEV)
    with torch.no_grad():
        eager = b(x)
        compiled = torch.compile(b, mode="max-autotune-no-cudagraphs", dynamic=False, fullgraph=True)
        out, code = run_and_get_code(compiled, x)
        assert "torch.ops.mstar_moe.moe_block" in "\n".join(code)
        # inductor may fuse the shared expert's gate differently from eager
        torch.testing.assert_close(out, eager, rtol=2e-2, atol=2e-3)
        first = out.clone()
        _capture_and_check(compiled, x, first)
