"""Fused q/k/v projection (+ q scaling) on gfx950 MFMA.

``prepare(module=, q_x=, kv_x=, apply_scale=, native=)`` is the
``Attention._prep_qkv`` hook of the reference
(python/fireprot/backends/amd/qkv_projection.py:54-66): for an eligible call
it returns q, k, v as ``[B, H, N, 32]`` views of one ``[3, B, N, 128]``
buffer, strides ``(N*128, 32, 128, 1)``, q multiplied by 1/sqrt(32);
otherwise ``native()``.
"""
from __future__ import annotations

import threading
from collections import Counter
from collections.abc import Callable
from typing import Any

from . import _native, switches
from .triangle_attention import ARCHITECTURE, HEAD_DIM, HEADS, _architecture

CHANNELS = 128
_lock = threading.RLock()
_counts: Counter[str] = Counter()


def qkv_projection(x: Any, wq: Any, wk: Any, wv: Any) -> Any:
    """``[3, *x.shape[:-1], 128]``: x @ W^T for W in (wq, wk, wv), q scaled."""
    import torch

    lib = _native.library()
    if not x.is_cuda or x.dtype != torch.float32 or not x.is_contiguous() or x.shape[-1] != CHANNELS:
        raise ValueError("x must be a contiguous float32 HIP tensor [..., 128]")
    for w in (wq, wk, wv):
        if (tuple(w.shape) != (CHANNELS, CHANNELS) or w.dtype != torch.float32
                or w.device != x.device or not w.is_contiguous()):
            raise ValueError("weights must be contiguous float32 [128, 128] on x's device")
    rows = x.numel() // CHANNELS
    out = torch.empty((3,) + tuple(x.shape), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        code = lib.fpx_qkv_projection(x.data_ptr(), rows, wq.data_ptr(), wk.data_ptr(),
                                      wv.data_ptr(), out.data_ptr(),
                                      torch.cuda.current_stream(x.device).cuda_stream)
    _native.check(code, "fpx_qkv_projection")
    return out


def supported(module: Any, q_x: Any, kv_x: Any, apply_scale: bool) -> bool:
    import torch

    if switches.disabled("FPX_DISABLE_QKV_PROJECTION"):
        return False
    if module.training or torch.is_grad_enabled() or not apply_scale:
        return False
    if getattr(module, "no_heads", None) != HEADS or getattr(module, "c_hidden", None) != HEAD_DIM:
        return False
    if not getattr(q_x, "is_cuda", False) or q_x.dim() != 3 or q_x.shape[-1] != CHANNELS:
        return False
    if (q_x.shape != kv_x.shape or q_x.stride() != kv_x.stride() or q_x.device != kv_x.device
            or q_x.dtype != kv_x.dtype or q_x.data_ptr() != kv_x.data_ptr()):
        return False
    if q_x.dtype != torch.float32 or not q_x.is_contiguous() or q_x.requires_grad:
        return False
    if q_x.data_ptr() % 16 or _architecture(q_x) != ARCHITECTURE:
        return False
    for linear in (module.linear_q, module.linear_k, module.linear_v):
        if getattr(linear, "bias", None) is not None or getattr(linear, "precision", None) is not None:
            return False
        if linear._forward_hooks or linear._forward_pre_hooks or "forward" in linear.__dict__:
            return False
        w = linear.weight
        if (tuple(w.shape) != (CHANNELS, CHANNELS) or w.dtype != torch.float32
                or w.device != q_x.device or not w.is_contiguous() or w.data_ptr() % 16):
            return False
    return _native.available()


def prepare(*, module: Any, q_x: Any, kv_x: Any, apply_scale: bool,
            native: Callable[[], Any]) -> Any:
    if not supported(module, q_x, kv_x, apply_scale):
        with _lock:
            _counts["fallback"] += 1
        return native()
    out = qkv_projection(q_x, module.linear_q.weight, module.linear_k.weight,
                         module.linear_v.weight)
    batch, length, _ = q_x.shape
    with _lock:
        _counts["hip"] += 1
    return tuple(t.view(batch, length, HEADS, HEAD_DIM).transpose(1, 2) for t in out.unbind(0))


def manifest() -> dict[str, Any]:
    with _lock:
        return {"counts": dict(_counts)}
