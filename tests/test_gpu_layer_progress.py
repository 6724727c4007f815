"""Forward progress of the one-launch decode layer kernel (stream_layer_kernel).

Its down phase waits for the gate_up work of its experts.  Before waiting,
a workgroup claims every unclaimed gate_up range that work depends on and
runs it itself, so a wait never depends on a workgroup that is not running.
These tests force the two rare cases from the host (a test mode read by the
launch; every kernel still exits normally):

* mode 1: odd workgroups skip claiming their own gate_up range, as if they
  were not resident yet; other workgroups must take those ranges over, and
  the output must be bit-identical to the normal launch's;
* mode 2: every down-phase wait gives up at once; the rows of the windows
  it gave up on must be NaN, the error word set and the failure counter
  raised: the output is invalid and reported, never silently wrong.

The reference has no such cross-workgroup wait (its five launches are
independent, mstar/utils/fused_moe/runner.py:118-158)."""
from __future__ import annotations

import ctypes
import contextlib

import pytest
import torch

from oracle import moe_oracle as O
from tests._util import assert_moe_close
from tests.test_gpu_stream import (DEV, E, H, I, K_TOP, _inputs, _ref, _route_quant, _stream_layer,
                                   layer_sync_words)

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def layer_mode(mode):
    from mstar_amd import _lib
    lib = _lib.load()
    _lib.check(lib.mstar_moe_debug_layer_test_mode(mode), "debug_layer_test_mode")
    try:
        yield
    finally:
        torch.cuda.synchronize()
        _lib.check(lib.mstar_moe_debug_layer_test_mode(0), "debug_layer_test_mode")


def _failures():
    from mstar_amd import _lib
    n = ctypes.c_int(-1)
    _lib.check(_lib.load().mstar_moe_layer_wait_failures(ctypes.byref(n)), "wait_failures")
    return n.value


def _claims(sync):
    base = (E + 16) // 16 * 16
    return sync[base::16].cpu()


def _layer_inputs(M, skewed):
    x, logits = _inputs(M, seed=500 + M)
    tw, ti, hq, hs = _route_quant(x, logits)
    if skewed:  # every token on experts 0-7: windows, and waits on many ranges
        g = torch.Generator().manual_seed(9)
        ti = torch.stack([torch.randperm(8, generator=g) for _ in range(M)]).int().to(DEV)
        tw = torch.softmax(torch.randn(M, K_TOP, generator=g), dim=-1).to(DEV)
    return x, tw, ti, hq, hs


def test_invalid_mode_is_rejected():
    from mstar_amd import _lib
    assert _lib.load().mstar_moe_debug_layer_test_mode(7) == 1


@pytest.mark.parametrize("M,skewed", [(32, False), (1, False), (64, False), (128, True)])
def test_unclaimed_ranges_are_taken_over(M, skewed):
    x, tw, ti, hq, hs = _layer_inputs(M, skewed)
    slots = M * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.empty(slots, H, dtype=torch.bfloat16, device=DEV)
    sync = _stream_layer(hq, hs, tw, ti, M, c2, c3)
    torch.cuda.synchronize()
    normal = _claims(sync)
    assert int(sync[E]) == 0
    assert int((normal == 2).sum()) == 0, "a range was taken over in a normal launch"
    ref3 = c3.clone()
    f0 = _failures()
    c2.fill_(0)
    c3.fill_(0)
    with layer_mode(1):
        sync = _stream_layer(hq, hs, tw, ti, M, c2, c3)
    claims = _claims(sync)
    assert int(sync[E]) == 0, "a down-phase wait gave up"
    assert _failures() == f0
    stolen = int((claims == 2).sum())
    assert stolen > 0, "no range was taken over"
    # Every range a workgroup ran was claimed once: owner (1) or thief (2).
    ran = claims[claims != 0]
    assert set(ran.tolist()) <= {1, 2}
    assert torch.equal(c3, ref3)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=DEV)
    from mstar_amd import ops
    ops.moe_sum_reduce(c3.view(M, K_TOP, H), out, 1.0)
    assert_moe_close(out, _ref(x, tw.cpu(), ti.cpu().long()), what=f"layer takeover M={M}")


@pytest.mark.parametrize("quant", ["fp8_w8a8", "w4a16"])
def test_moe_layer_takeover_bit_identical(quant):
    """The same through mstar_moe_layer (routing launch clears the claim
    words), FP8 and W4A16."""
    from mstar_amd import _lib, ops
    from mstar_amd import quant as Q
    g = torch.Generator().manual_seed(31)
    w1 = (torch.randn(E, 2 * I, H, generator=g) * 0.02).to(DEV)
    w2 = (torch.randn(E, H, I, generator=g) * 0.02).to(DEV)
    if quant == "fp8_w8a8":
        q1, s1 = Q.quantize_fp8_block(w1)
        q2, s2 = Q.quantize_fp8_block(w2)
        qc = _lib.QUANT_FP8_W8A8
    else:
        q1, s1 = Q.quantize_int4_group(w1)
        q2, s2 = Q.quantize_int4_group(w2)
        qc = _lib.QUANT_W4A16
    x = torch.randn(32, H, generator=g).to(torch.bfloat16).to(DEV)
    logits = torch.randn(32, E, generator=g).to(DEV)
    ref, _, _ = ops.moe_layer(x, logits, q1, q2, K_TOP, True, 0, qc, s1, s2)
    f0 = _failures()
    with layer_mode(1):
        for _ in range(3):
            out, _, _ = ops.moe_layer(x, logits, q1, q2, K_TOP, True, 0, qc, s1, s2)
            torch.cuda.synchronize()
            assert torch.equal(out, ref)
    assert _failures() == f0


def test_wait_give_up_is_reported_and_poisons():
    M = 32
    x, tw, ti, hq, hs = _layer_inputs(M, False)
    slots = M * K_TOP
    c2 = torch.empty(slots, I, dtype=torch.bfloat16, device=DEV)
    c3 = torch.zeros(slots, H, dtype=torch.bfloat16, device=DEV)
    f0 = _failures()
    with layer_mode(2):
        sync = _stream_layer(hq, hs, tw, ti, M, c2, c3)
    assert int(sync[E]) == 1, "the error word was not set"
    assert _failures() > f0
    assert bool(torch.isnan(c3.float()).all()), "rows of a window that gave up are not NaN"
    # The next normal launch is valid again.
    sync = _stream_layer(hq, hs, tw, ti, M, c2, c3)
    torch.cuda.synchronize()
    assert int(sync[E]) == 0
    assert not bool(torch.isnan(c3.float()).any())
