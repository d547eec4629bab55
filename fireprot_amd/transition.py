"""Pair transition on gfx950: ``Transition.forward`` (n = 4, c_in = 128).

Drop-in for the reference's ``dispatch_transition(module=, x=, native=)``
(python/fireprot/backends/amd/recycle.py:360-390), which the Protenix hooks
install on ``Transition.forward`` (python/fireprot/adapters/protenix/
hooks.py:56-68).  The HIP candidate runs the whole transition as one C-ABI
call, ``fpx_transition``: LayerNorm, the SiLU-gated 128 -> 512 dual
projection (the reference's ``transition_projection``, recycle.py:214-220)
and the 512 -> 128 ``linear_no_bias`` (recycle.py:226), for any row count and
strided inputs.  ``pair_transition_residual`` additionally folds the
Pairformer's ``z = z + transition(z)`` into the output store.  There is no
CPU path: unsupported calls go to the caller's ``native`` function.
"""
from __future__ import annotations

import dataclasses
import functools
from collections.abc import Callable
from typing import Any

import torch

from . import _native, switches
from . import workspace as ws_cache
from .registry import OperationSignature, registry, signature_from_tensor

OPERATION = "gated_transition"
IMPLEMENTATION = "amd-gfx950-hip-transition-f32"
ARCHITECTURE = "gfx950"
CHANNELS = 128
EXPANSION = 4


@dataclasses.dataclass
class TransitionWeights:
    """``layernorm1`` affine (nullable), ``w_a``/``w_b`` ``[512, 128]``,
    ``w_o`` ``[128, 512]``, float32 and contiguous."""

    ln_w: torch.Tensor | None
    ln_b: torch.Tensor | None
    w_a: torch.Tensor
    w_b: torch.Tensor
    w_o: torch.Tensor
    eps: float = 1e-5

    @classmethod
    def from_tensors(cls, *, ln_w, ln_b, w_a, w_b, w_o, eps: float = 1e-5) -> "TransitionWeights":
        def prep(t):
            return None if t is None else t.detach().to(torch.float32).contiguous()
        return cls(prep(ln_w), prep(ln_b), prep(w_a), prep(w_b), prep(w_o), float(eps))

    @classmethod
    def from_module(cls, module: Any) -> "TransitionWeights":
        """Protenix ``Transition``: ``layernorm1``, ``linear_no_bias_a``,
        ``linear_no_bias_b``, ``linear_no_bias`` (recycle.py:210-226)."""
        for layer in (module.linear_no_bias_a, module.linear_no_bias_b, module.linear_no_bias):
            if getattr(layer, "bias", None) is not None:
                raise ValueError("transition projections must be bias-free")
        norm = module.layernorm1
        return cls.from_tensors(ln_w=getattr(norm, "weight", None), ln_b=getattr(norm, "bias", None),
                                w_a=module.linear_no_bias_a.weight,
                                w_b=module.linear_no_bias_b.weight,
                                w_o=module.linear_no_bias.weight,
                                eps=float(getattr(norm, "eps", 1e-5)))

    def to(self, device: Any) -> "TransitionWeights":
        moved = {f.name: getattr(self, f.name) for f in dataclasses.fields(self)}
        return TransitionWeights(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v)
                                    for k, v in moved.items()})


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _rows(t: torch.Tensor) -> tuple[int, int, int, int] | None:
    """(rows_i, rows_j, stride_i, stride_j) addressing t's 128-channel rows, or
    None when t's layout has no such two-index form."""
    if t.shape[-1] != CHANNELS or t.stride(-1) != 1:
        return None
    if t.dim() == 3:
        return t.shape[0], t.shape[1], t.stride(0), t.stride(1)
    if t.dim() == 2:
        return 1, t.shape[0], 0, t.stride(0)
    if t.is_contiguous():
        rows = t.numel() // CHANNELS
        return 1, rows, 0, CHANNELS
    return None


def transition(x: torch.Tensor, weights: TransitionWeights, *, out: torch.Tensor | None = None,
               accumulate: bool = False, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One ``fpx_transition`` call on x's device and current stream.

    ``x`` is ``[..., 128]`` float32 (3-D with row strides in multiples of 4
    floats and a 16-byte aligned start, otherwise copied contiguous first);
    the result has x's shape.  ``out=x, accumulate=True`` is the
    in-place ``x += transition(x)``.
    """
    if not x.is_cuda or x.dtype != torch.float32:
        raise ValueError("x must be a float32 tensor on a HIP device")
    src = _rows(x)
    if src is None or src[2] % 4 or src[3] % 4 or x.data_ptr() % 16:
        x = x.contiguous()
        if x.data_ptr() % 16:  # contiguous already, at a misaligned offset
            x = x.clone()
        src = _rows(x)
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float32, device=x.device)
    dst = _rows(out)
    if dst is None or tuple(out.shape) != tuple(x.shape) or out.dtype != torch.float32:
        raise ValueError("out must be float32 with x's shape and addressable rows")
    lib = _native.library()
    size = lib.fpx_transition_workspace_bytes(src[0], src[1], CHANNELS, EXPANSION)
    if size == 0:
        raise ValueError(f"unsupported transition row count {src[0]} x {src[1]}")
    if workspace is None or workspace.numel() < size:
        workspace = torch.empty(size, dtype=torch.uint8, device=x.device)
    w = weights
    with torch.cuda.device(x.device):
        code = lib.fpx_transition(
            x.data_ptr(), src[0], src[1], src[2], src[3], _ptr(w.ln_w), _ptr(w.ln_b), w.eps,
            w.w_a.data_ptr(), w.w_b.data_ptr(), w.w_o.data_ptr(), CHANNELS, EXPANSION,
            int(bool(accumulate)), out.data_ptr(), dst[2], dst[3], workspace.data_ptr(),
            workspace.numel(), torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_transition")
    return out


def pair_transition_residual(z: torch.Tensor, weights: TransitionWeights,
                             workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``z += transition(z)`` in place (the Pairformer's pair-transition step)."""
    return transition(z, weights, out=z, accumulate=True, workspace=workspace)


# ------------------------------------------------------------ dispatch

@functools.lru_cache(maxsize=None)
def _device_architecture(index: int) -> str:
    properties = torch.cuda.get_device_properties(index)
    return str(getattr(properties, "gcnArchName", "")).split(":", 1)[0]


def _architecture(tensor: Any) -> str:
    try:
        if tensor.device.type != "cuda":
            return "cpu"
        return _device_architecture(int(tensor.device.index or 0))
    except Exception:
        return "unknown"


def eligible(module: Any, x: Any) -> tuple[bool, str]:
    if not getattr(x, "is_cuda", False) or x.dtype != torch.float32:
        return False, "x is not a float32 HIP tensor"
    if x.dim() < 1 or x.shape[-1] != CHANNELS or x.numel() == 0:
        return False, "x must be [..., 128] and non-empty"
    if getattr(module, "n", None) != EXPANSION or getattr(module, "c_in", None) != CHANNELS:
        return False, "transition must have n = 4 and c_in = 128"
    try:
        layers = (module.linear_no_bias_a, module.linear_no_bias_b, module.linear_no_bias)
        norm = module.layernorm1
    except AttributeError as error:
        return False, f"module layout: {error}"
    shapes = ((EXPANSION * CHANNELS, CHANNELS),) * 2 + ((CHANNELS, EXPANSION * CHANNELS),)
    for layer, shape in zip(layers, shapes):
        weight = getattr(layer, "weight", None)
        if not isinstance(weight, torch.Tensor) or tuple(weight.shape) != shape:
            return False, "projection weights have the wrong shape"
        if weight.device != x.device or getattr(layer, "bias", None) is not None:
            return False, "projection weights must be bias-free on x's device"
    for t in (getattr(norm, "weight", None), getattr(norm, "bias", None)):
        if t is not None and t.device != x.device:
            return False, "LayerNorm parameters are not on x's device"
    return True, ""


def _supports(signature: OperationSignature) -> bool | tuple[bool, str]:
    if (off := switches.rejection("FPX_DISABLE_TRANSITION")) is not None:
        return off
    attributes = dict(signature.attributes)
    if signature.device_type != "cuda":
        return False, "device is not CUDA/HIP"
    if signature.architecture != ARCHITECTURE:
        return False, f"architecture is not {ARCHITECTURE}"
    if signature.dtype != "float32":
        return False, "dtype is not float32"
    if signature.mode != "inference":
        return False, "training or autograd is enabled"
    if attributes.get("expansion") != "4":
        return False, "transition expansion is not four"
    if attributes.get("eligible") != "True":
        return False, attributes.get("reason", "tensor/module contract mismatch")
    if not _native.available():
        return False, "HIP extension unavailable"
    return True


def _hip(*, module: Any, x: Any, native: Callable[..., Any]) -> Any:
    del native
    src = _rows(x)
    size = (_native.library().fpx_transition_workspace_bytes(src[0], src[1], CHANNELS, EXPANSION)
            if src is not None else 0)
    ws = ws_cache.get(x.device, size, purpose="transition") if size else None
    return transition(x, TransitionWeights.from_module(module).to(x.device), workspace=ws)


def dispatch_transition(*, module: Any, x: Any, native: Callable[..., Any]) -> Any:
    """Select the HIP transition or the caller's native function (same keyword
    contract as the reference's ``dispatch_transition``)."""
    mode = ("inference" if not getattr(module, "training", False) and not torch.is_grad_enabled()
            and not getattr(x, "requires_grad", False) else "training")
    ok, reason = eligible(module, x)
    signature = signature_from_tensor(
        OPERATION, x, architecture=_architecture(x), mode=mode, mask="none", inplace=False,
        attributes={"expansion": getattr(module, "n", None), "c_in": getattr(module, "c_in", None),
                    "eligible": ok, "reason": reason})
    return registry.dispatch(signature, native, module=module, x=x, native=native)


registry.register(operation=OPERATION, name=IMPLEMENTATION, function=_hip, supports=_supports,
                  priority=40, version="1")
