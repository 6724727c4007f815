"""The reference's native op under its own name: ``torch.ops._mstar_moe_C``.

The reference's C++ extension defines one op,

    TORCH_LIBRARY(_mstar_moe_C, m)
      moe_align_block_size(Tensor topk_ids, int num_experts, int block_size,
                           Tensor! sorted_token_ids, Tensor! experts_ids,
                           Tensor! num_tokens_post_pad) -> ()

(mstar/utils/fused_moe/csrc/moe_align_block_size.cu:273-282), which
``moe_align_block_size`` (mstar/utils/fused_moe/align.py:55-103) calls on
buffers it allocates itself (align.py:78-87).  :func:`register` defines that
op, with the same schema, on this library's ``mstar_moe_align_block_size``,
so the reference's Python code runs unchanged once this module is imported in
place of its extension.

Behaviour kept from the reference op:

* ``topk_ids`` must be int32 (``TORCH_CHECK``, .cu:210-211);
* the expert count rounded up to 32 must be below 1024 (.cu:221-224);
* the outputs are written in place; the scratch the op needs (the reference's
  ``cumsum_buffer``, .cu:228-230) comes from torch's caching allocator;
* every failure raises ``RuntimeError``, as ``TORCH_CHECK`` does.
"""
from __future__ import annotations

import ctypes
import threading

import torch

from . import _lib

NAMESPACE = "_mstar_moe_C"
SCHEMA = ("moe_align_block_size(Tensor topk_ids, int num_experts, int block_size, "
          "Tensor! sorted_token_ids, Tensor! experts_ids, Tensor! num_tokens_post_pad) -> ()")

_lock = threading.Lock()
_registered = False
_library = None  # keeps the torch.library.Library (and so the definition) alive


def _align_impl(topk_ids: torch.Tensor, num_experts: int, block_size: int,
                sorted_token_ids: torch.Tensor, experts_ids: torch.Tensor,
                num_tokens_post_pad: torch.Tensor) -> None:
    if topk_ids.dtype != torch.int32:
        raise RuntimeError("moe_align_block_size: topk_ids must be int32")
    for name, t in (("sorted_token_ids", sorted_token_ids), ("experts_ids", experts_ids),
                    ("num_tokens_post_pad", num_tokens_post_pad)):
        if t.dtype != torch.int32 or not t.is_contiguous() or t.device != topk_ids.device:
            raise RuntimeError(f"moe_align_block_size: {name} must be a contiguous int32 "
                               f"tensor on {topk_ids.device}")
    if not topk_ids.is_cuda:
        raise RuntimeError("moe_align_block_size: topk_ids must be a GPU tensor")
    if num_tokens_post_pad.numel() < 1:
        raise RuntimeError("moe_align_block_size: num_tokens_post_pad needs one element")
    ids = topk_ids.contiguous()
    lib = _lib.load()
    need = ctypes.c_size_t()
    rc = lib.mstar_moe_align_scratch_size(ids.numel(), int(num_experts), ctypes.byref(need))
    if rc != 0:
        raise RuntimeError(lib.mstar_moe_last_error().decode(errors="replace"))
    scratch = (torch.empty(need.value, dtype=torch.uint8, device=ids.device)
               if need.value else None)
    with torch.cuda.device(ids.device):
        rc = lib.mstar_moe_align_block_size(
            ids.data_ptr(), _lib.DT_I32, ids.numel(), int(num_experts), int(block_size),
            sorted_token_ids.data_ptr(), sorted_token_ids.numel(),
            experts_ids.data_ptr(), experts_ids.numel(), num_tokens_post_pad.data_ptr(),
            None, None, _lib.ptr(scratch), need.value, _lib.stream_of(ids))
    if rc != 0:
        raise RuntimeError(lib.mstar_moe_last_error().decode(errors="replace"))


def register() -> None:
    """Define ``torch.ops._mstar_moe_C.moe_align_block_size`` (once per process).

    Raises ``RuntimeError`` if another library (the reference's own
    extension) already defined the namespace's op."""
    global _registered, _library
    with _lock:
        if _registered:
            return
        lib = torch.library.Library(NAMESPACE, "DEF")
        lib.define(SCHEMA)
        lib.impl("moe_align_block_size", _align_impl, "CUDA")
        _library = lib
        _registered = True


def is_registered() -> bool:
    return _registered
