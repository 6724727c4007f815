"""mstar_moe_layer_noalloc (the layer with its workspace in a fixed device
array) against mstar_moe_layer with a caller workspace, through the C-ABI:
bit-identical outputs, routing weights and ids, on two calls in a row with
the second smaller (the array keeps the first call's contents), and a clear
rejection of sizes past the array."""
from __future__ import annotations

import ctypes

import pytest
import torch

from tests.test_gpu_moe import _fp8_weights, _hidden, _weights

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _call(lib, fn, x, logits, w1, w2, s1, s2, k, quant, ws=None):
    from mstar_amd import _lib
    M, H = x.shape
    E = w1.shape[0]
    inter = w2.shape[2] * (8 if quant == _lib.QUANT_W4A16 else 1)
    out = torch.full((M, H), float("nan"), dtype=x.dtype, device=DEV)
    tw = torch.full((M, k), -1.0, dtype=torch.float32, device=DEV)
    ti = torch.full((M, k), -1, dtype=torch.int64, device=DEV)
    args = [_lib.ptr(x), _lib.dtype_code(x.dtype), M, H, _lib.ptr(logits),
            _lib.dtype_code(logits.dtype), 1, _lib.ptr(w1), _lib.ptr(w2), E, inter, quant,
            _lib.ptr(s1), _lib.ptr(s2), k, 0, _lib.ptr(out), _lib.ptr(tw), _lib.ptr(ti)]
    if ws is not None:
        args += [_lib.ptr(ws), ws.numel()]
    st = getattr(lib, fn)(*args, _lib.stream_of(x))
    return st, out, tw, ti


def _workspace(lib, M, H, E, inter, k, quant, dt):
    from mstar_amd import _lib
    n = ctypes.c_size_t(0)
    _lib.check(lib.mstar_moe_layer_workspace_size(M, H, E, inter, k, quant, dt, ctypes.byref(n)), "ws")
    return torch.empty(max(n.value, 1), dtype=torch.uint8, device=DEV)


@pytest.mark.parametrize("quant_name,Ms", [("fp8", (32, 4)), ("fp8", (256, 65)),
                                           ("none", (200, 7)), ("w4a16", (64, 1))])
def test_noalloc_layer_matches_workspace_layer(quant_name, Ms):
    from mstar_amd import _lib
    from mstar_amd import quant as Q
    lib = _lib.load()
    H, E, I, k = 2048, 128, 768, 8
    if quant_name == "fp8":
        quant = _lib.QUANT_FP8_W8A8
        w1, s1, w2, s2 = _fp8_weights(H, E, I)
    elif quant_name == "w4a16":
        quant = _lib.QUANT_W4A16
        b1, b2 = _weights(H, E, I)
        w1, s1 = Q.quantize_int4_group(b1)
        w2, s2 = Q.quantize_int4_group(b2)
    else:
        quant = _lib.QUANT_NONE
        w1, w2 = _weights(H, E, I)
        s1 = s2 = None
    for M in Ms:  # second call smaller: the array still holds the first call's data
        print(f"noalloc {quant_name} M={M}", flush=True)
        x = _hidden(M, H, seed=M + 3).to(DEV)
        logits = torch.randn(M, E, generator=torch.Generator().manual_seed(M)).to(DEV)
        ws = _workspace(lib, M, H, E, I, k, quant, _lib.DT_BF16)
        st0, o0, w0, i0 = _call(lib, "mstar_moe_layer", x, logits, w1, w2, s1, s2, k, quant, ws)
        st1, o1, w1_, i1 = _call(lib, "mstar_moe_layer_noalloc", x, logits, w1, w2, s1, s2, k, quant)
        torch.cuda.synchronize()
        assert st0 == 0, lib.mstar_moe_last_error()
        assert st1 == 0, lib.mstar_moe_last_error()
        assert torch.equal(i1, i0) and torch.equal(w1_, w0)
        assert torch.equal(o1.view(torch.int16), o0.view(torch.int16))


def test_noalloc_rejects_sizes_past_the_array():
    from mstar_amd import _lib
    lib = _lib.load()
    H, E, I, k, M = 2048, 128, 768, 8, 2048
    n = ctypes.c_size_t(0)
    assert lib.mstar_moe_layer_workspace_size(M, H, E, I, k, _lib.QUANT_FP8_W8A8, _lib.DT_BF16,
                                              ctypes.byref(n)) == 0
    assert n.value > (16 << 20)
    w1, s1, w2, s2 = _fp8_weights(H, E, I)
    x = torch.zeros(M, H, dtype=torch.bfloat16, device=DEV)
    logits = torch.zeros(M, E, device=DEV)
    st, out, _, _ = _call(lib, "mstar_moe_layer_noalloc", x, logits, w1, w2, s1, s2, k,
                          _lib.QUANT_FP8_W8A8)
    torch.cuda.synchronize()
    assert st == 4
    assert b"more than the" in lib.mstar_moe_last_error()
    assert torch.isnan(out.float()).all()  # nothing launched
