"""C-ABI checks that need no GPU: the library loads, exports exactly the
entry points include/mstar_moe.h declares, the Python binding declares the
same set, and argument validation fails cleanly (status + message) before
anything is launched."""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest
import torch

from mstar_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mstar_moe.h")


def header_functions() -> list[str]:
    text = open(HEADER).read()
    return re.findall(r"^(?:const\s+)?\w+\*?\s+\*?(mstar_\w+)\(", text, flags=re.M)


def test_header_parses():
    names = header_functions()
    assert "mstar_fused_moe" in names and "mstar_moe_align_block_size" in names
    assert len(names) == len(set(names))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (mstar_\w+)", out))
    assert exported == set(header_functions())


def test_binding_matches_header():
    assert list(_lib.SIGNATURES) == header_functions()


def test_abi_version():
    assert _lib.load().mstar_moe_abi_version() == 1


def _err():
    return _lib.load().mstar_moe_last_error().decode()


def test_align_rejects_too_many_experts():
    lib = _lib.load()
    st = lib.mstar_moe_align_block_size(None, _lib.DT_I32, 0, 1024, 16, None, 0, None, 0, None,
                                        None, None, None, 0, None)
    assert st == 1 and "less than 1024" in _err()


def test_align_rejects_small_output():
    lib = _lib.load()
    buf = ctypes.c_void_p(8)  # never dereferenced: validation fails first
    st = lib.mstar_moe_align_block_size(buf, _lib.DT_I32, 256, 128, 16, buf, 100, buf, 1000, buf,
                                        None, None, None, 0, None)
    assert st == 1 and "too small" in _err()


def test_fused_moe_workspace_and_shape_checks():
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    assert lib.mstar_fused_moe_workspace_size(32, 2048, 128, 768, 8, _lib.QUANT_FP8_W8A8,
                                              _lib.DT_BF16, 1, ctypes.byref(n)) == 0
    assert n.value > 32 * 8 * 768 * 2
    # quantised paths need multiples of 128; the bf16 path takes any size
    assert lib.mstar_fused_moe_workspace_size(32, 2000, 128, 768, 8, _lib.QUANT_FP8_W8A8,
                                              _lib.DT_BF16, 1, ctypes.byref(n)) == 2
    assert "multiples of 128" in _err()
    assert lib.mstar_fused_moe_workspace_size(32, 2000, 128, 100, 8, 0, _lib.DT_BF16, 1,
                                              ctypes.byref(n)) == 0
    assert n.value >= 32 * 8 * 100 * 2 + 32 * 8 * 2000 * 2
    assert lib.mstar_fused_moe_workspace_size(32, 2048, 128, 768, 200, 0, _lib.DT_BF16, 1,
                                              ctypes.byref(n)) == 1
    # fp16 activations are not accepted by the quantised paths
    assert lib.mstar_fused_moe_workspace_size(32, 2048, 128, 768, 8, _lib.QUANT_W4A16,
                                              _lib.DT_F16, 1, ctypes.byref(n)) == 2


def test_workspace_too_small_is_reported():
    lib = _lib.load()
    p = ctypes.c_void_p(256)
    st = lib.mstar_fused_moe(p, _lib.DT_BF16, 32, 2048, p, p, 128, 768, 0, None, None, p,
                             _lib.DT_F32, p, _lib.DT_I32, 8, 0, 1, p, p, 16, None)
    assert st == 4 and "workspace too small" in _err()


def test_layer_and_route_sizes():
    lib = _lib.load()
    n = ctypes.c_size_t(0)
    assert lib.mstar_moe_layer_workspace_size(32, 2048, 128, 768, 8, _lib.QUANT_FP8_W8A8,
                                              _lib.DT_BF16, ctypes.byref(n)) == 0
    assert n.value > 0
    assert lib.mstar_moe_route_scratch_size(8192, 128, 8, ctypes.byref(n)) == 0
    assert n.value >= 64 * 128 * 4
    assert lib.mstar_moe_align_scratch_size(65536, 128, ctypes.byref(n)) == 0
    assert n.value == 64 * 128 * 4
    p = ctypes.c_void_p(256)
    st = lib.mstar_moe_route(p, _lib.DT_F32, 8192, 128, 8, 1, p, None, None, 64, p, 100, p, 10, p,
                             None, None, None, 0, None)
    assert st == 1 and "too small" in _err()


def test_topk_rejects_bad_k():
    st = _lib.load().mstar_moe_topk_softmax(None, _lib.DT_F32, 4, 8, 9, 1, None, None, None, None)
    assert st == 1


def test_quant_rejects_group_size():
    st = _lib.load().mstar_quant_fp8_per_token_group(None, _lib.DT_BF16, 4, 256, 64, None, None, None)
    assert st == 2


def test_fp8_mm_rejects_unaligned_k():
    p = ctypes.c_void_p(256)
    st = _lib.load().mstar_fp8_scaled_mm(p, p, p, p, p, 4, 16, 100, None)
    assert st == 1


def test_python_ops_refuse_cpu_tensors():
    from mstar_amd.fused_moe import fused_experts, moe_align_block_size
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    w1 = torch.zeros(2, 256, 128, dtype=torch.bfloat16)
    w2 = torch.zeros(2, 128, 128, dtype=torch.bfloat16)
    tw = torch.ones(4, 1)
    ti = torch.zeros(4, 1, dtype=torch.int64)
    with pytest.raises(ValueError, match="GPU"):
        fused_experts(x, w1, w2, tw, ti)
    with pytest.raises(ValueError, match="GPU"):
        moe_align_block_size(ti.int(), 16, 2)


def test_get_default_config_matches_reference_rule():
    from mstar_amd.fused_moe import get_default_config
    from oracle.moe_oracle import get_default_config as ref
    for M in (1, 32, 128, 129, 8192):
        assert get_default_config(M, 128, 1536, 2048, 8) == ref(M, 128)
