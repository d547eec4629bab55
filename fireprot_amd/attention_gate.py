"""Sigmoid output gate of ``Attention._wrap_up`` on gfx950.

``wrap_up(module=, o=, x=, native=)`` is the reference hook
(python/fireprot/backends/amd/attention_gate.py:28-56):
``linear_o(o * sigmoid(linear_g(x)))`` with the gate multiply in the HIP
kernel ``fpx_sigmoid_mul_out`` (out of place, inputs untouched) and the two
linears left to the module.  Inside the full block the gate is instead fused
into the attention epilogue.
"""
from __future__ import annotations

import threading
from collections import Counter
from collections.abc import Callable
from typing import Any

from . import _native, switches
from .triangle_attention import ARCHITECTURE, HEAD_DIM, HEADS, _architecture

_lock = threading.RLock()
_counts: Counter[str] = Counter()


def sigmoid_mul_out(gate: Any, value: Any) -> Any:
    """``value * sigmoid(gate)`` into a new tensor; HIP only."""
    import torch

    lib = _native.library()
    if (gate.shape != value.shape or gate.dtype != torch.float32 or value.dtype != torch.float32
            or not gate.is_cuda or gate.device != value.device):
        raise ValueError("gate and value must be float32 HIP tensors of one shape")
    if not gate.is_contiguous() or not value.is_contiguous() or gate.numel() % 4:
        raise ValueError("gate and value must be contiguous with numel % 4 == 0")
    out = torch.empty_like(value)
    with torch.cuda.device(value.device):
        code = lib.fpx_sigmoid_mul_out(gate.data_ptr(), value.data_ptr(), out.data_ptr(),
                                       value.numel(),
                                       torch.cuda.current_stream(value.device).cuda_stream)
    _native.check(code, "fpx_sigmoid_mul_out")
    return out


def supported(module: Any, o: Any, x: Any) -> bool:
    import torch

    if switches.disabled("FPX_DISABLE_ATTENTION_GATE"):
        return False
    if module.training or torch.is_grad_enabled():
        return False
    if getattr(module, "linear_g", None) is None:
        return False
    if getattr(module, "no_heads", None) != HEADS or getattr(module, "c_hidden", None) != HEAD_DIM:
        return False
    if not getattr(x, "is_cuda", False) or x.device != o.device or _architecture(x) != ARCHITECTURE:
        return False
    if tuple(o.shape) != tuple(x.shape[:-1]) + (HEADS, HEAD_DIM) or x.shape[-1] != HEADS * HEAD_DIM:
        return False
    if any(t.dtype != torch.float32 or not t.is_contiguous() or t.requires_grad
           or t.data_ptr() % 16 for t in (x, o)):
        return False
    return _native.available()


def wrap_up(*, module: Any, o: Any, x: Any, native: Callable[[], Any]) -> Any:
    if not supported(module, o, x):
        with _lock:
            _counts["fallback"] += 1
        return native()
    gate = module.linear_g(x)
    gated = sigmoid_mul_out(gate, o.reshape(gate.shape))
    with _lock:
        _counts["hip"] += 1
    return module.linear_o(gated)


def manifest() -> dict[str, Any]:
    with _lock:
        return {"counts": dict(_counts)}
