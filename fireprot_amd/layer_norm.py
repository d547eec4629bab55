"""C128 pair LayerNorm on gfx950, contiguous or transposed view, one kernel.

``dispatch_layer_norm(module=, x=, native=)`` has the reference's hook
signature (python/fireprot/backends/amd/recycle.py:293-357): eligible calls
run ``fpx_layer_norm_c128``, everything else calls ``native()``.  The kernel
reads rows through two strides, so the ending node's ``z.transpose(0, 1)``
view (strides ``(128, N*128, 1)``) needs no contiguous copy -- the job of the
reference's separate transposed kernel (kernels/amd/fireprot_amd_ops.cu:
957-1104).  The output is always contiguous.
"""
from __future__ import annotations

import threading
from collections import Counter
from collections.abc import Callable
from typing import Any

from . import _native, switches
from .triangle_attention import ARCHITECTURE, _architecture

CHANNELS = 128
_lock = threading.RLock()
_counts: Counter[str] = Counter()


def _rows(x: Any) -> tuple[int, int, int, int]:
    if x.dim() == 3:
        return x.shape[0], x.shape[1], x.stride(0), x.stride(1)
    if x.dim() == 2:
        return 1, x.shape[0], 0, x.stride(0)
    raise ValueError("x must be [A, B, 128] or [R, 128]")


def layer_norm_c128(x: Any, weight: Any, bias: Any, eps: float) -> Any:
    """LayerNorm over the last (128) axis of a 2-D or 3-D view; HIP only."""
    import torch

    lib = _native.library()
    if not x.is_cuda or x.dtype != torch.float32 or x.shape[-1] != CHANNELS or x.stride(-1) != 1:
        raise ValueError("x must be a float32 HIP tensor [..., 128] with unit channel stride")
    rows_i, rows_j, stride_i, stride_j = _rows(x)
    for t in (weight, bias):
        if t is not None and (tuple(t.shape) != (CHANNELS,) or t.dtype != torch.float32
                              or t.device != x.device or not t.is_contiguous()):
            raise ValueError("weight/bias must be contiguous float32 [128] on x's device")
    y = torch.empty(tuple(x.shape), device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        code = lib.fpx_layer_norm_c128(
            x.data_ptr(), rows_i, rows_j, stride_i, stride_j,
            None if weight is None else weight.data_ptr(),
            None if bias is None else bias.data_ptr(), float(eps), y.data_ptr(),
            torch.cuda.current_stream(x.device).cuda_stream)
    _native.check(code, "fpx_layer_norm_c128")
    return y


def eligible(module: Any, x: Any) -> tuple[bool, str]:
    import torch

    if (off := switches.rejection("FPX_DISABLE_LAYER_NORM")) is not None:
        return off
    if getattr(x, "device", None) is None or x.device.type != "cuda":
        return False, "device is not CUDA/HIP"
    if _architecture(x) != ARCHITECTURE:
        return False, f"architecture is not {ARCHITECTURE}"
    if x.dtype != torch.float32:
        return False, "dtype is not float32"
    if module.training or torch.is_grad_enabled() or x.requires_grad:
        return False, "training or autograd is enabled"
    if x.dim() not in (2, 3) or x.shape[-1] != CHANNELS or x.stride(-1) != 1:
        return False, "input is not [..., 128] with unit channel stride"
    rows_i, rows_j, stride_i, stride_j = _rows(x)
    if stride_i % 2 or stride_j % 2 or x.data_ptr() % 8:
        return False, "rows are not 8-byte aligned"
    if tuple(getattr(module, "normalized_shape", (CHANNELS,))) != (CHANNELS,):
        return False, "normalized shape is not (128,)"
    for t in (module.weight, module.bias):
        if t is not None and (t.dtype != torch.float32 or t.device != x.device):
            return False, "affine parameters are not float32 on x's device"
    if not _native.available():
        return False, "HIP extension unavailable"
    return True, ""


def dispatch_layer_norm(*, module: Any, x: Any, native: Callable[[], Any]) -> Any:
    ok, _ = eligible(module, x)
    if not ok:
        with _lock:
            _counts["native"] += 1
        return native()
    layout = "transposed" if x.dim() == 3 and x.stride(0) < x.stride(1) else "rows"
    with _lock:
        _counts[f"hip-{layout}"] += 1
    weight = None if module.weight is None else module.weight.contiguous()
    bias = None if module.bias is None else module.bias.contiguous()
    return layer_norm_c128(x, weight, bias, module.eps)


def manifest() -> dict[str, Any]:
    with _lock:
        return {"counts": dict(_counts)}
