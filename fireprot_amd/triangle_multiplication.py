"""Triangle multiplicative update (outgoing / incoming) on gfx950.

Drop-in for the Protenix ``TriangleMultiplicativeUpdate.forward`` branch
``triangle_multiplicative="fireprot"`` (patches/protenix/0001-*.patch:14-46):
``dispatch_triangle_multiplication`` has the reference's keyword signature
and signature attributes (python/fireprot/backends/amd/
triangle_multiplication.py:377-418) and registers one candidate in the shared
registry.  The candidate runs the whole update as one C-ABI call,
``fpx_tri_mul`` (include/fireprot_amd.h):

* LayerNorm_in, the four gated projections and the mask are fused and write
  ``a``, ``b`` channel-blocked, one contiguous 2 KB block per wave and
  32-key tile, with each (channel, row)'s max |value| (the reference's
  sigmoid-pack step, triangle_multiplication.py:301-316);
* the per-channel contraction is a hand-written batched GEMM on the 16-bit
  matrix cores with FP32 accuracy (power-of-two scaled fp16 hi/lo planes,
  three terms; the reference's library BMM, ``packed_bmm``, :318);
* LayerNorm_out, ``linear_z``, ``sigmoid(linear_g(LN_in z))`` and the
  residual are fused into one epilogue kernel (:321-339), which writes into
  ``z`` in place.

In-place contract (triangle_multiplication.py:73-92): with ``inplace_safe``
the result is written into ``z`` -- ``z + update`` when ``add_with_inplace``,
``update`` otherwise -- and ``z`` is returned; without it a new update tensor
is returned.  Unlike the reference, any N <= 4096 and explicit masks are
accepted.  There is no CPU path: unsupported calls go to the caller's
``native`` function.
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

OPERATION = "triangle_multiplication"
IMPLEMENTATION = "amd-gfx950-hip-triangle-multiplication-f32"
ARCHITECTURE = "gfx950"
CHANNELS = 128
MAX_N = 4096
LINEARS = ("linear_a_p", "linear_a_g", "linear_b_p", "linear_b_g", "linear_z", "linear_g")


@dataclasses.dataclass
class TriMulWeights:
    """Device-resident weights of one update, torch ``[out, in]``.

    ``w_abpg`` stacks W_a_p, W_a_g, W_b_p, W_b_g into ``[512, 128]``;
    ``b_abpg`` their biases ``[512]`` or None.
    """

    ln_in_w: torch.Tensor | None
    ln_in_b: torch.Tensor | None
    w_abpg: torch.Tensor
    b_abpg: torch.Tensor | None
    ln_out_w: torch.Tensor | None
    ln_out_b: torch.Tensor | None
    w_z: torch.Tensor
    b_z: torch.Tensor | None
    w_g: torch.Tensor
    b_g: torch.Tensor | None
    eps_in: float = 1e-5
    eps_out: float = 1e-5

    @classmethod
    def from_tensors(cls, *, ln_in_w, ln_in_b, w_a_p, w_a_g, w_b_p, w_b_g, ln_out_w, ln_out_b,
                     w_z, w_g, b_a_p=None, b_a_g=None, b_b_p=None, b_b_g=None, b_z=None,
                     b_g=None, eps_in: float = 1e-5, eps_out: float = 1e-5) -> "TriMulWeights":
        def prep(t):
            return None if t is None else t.detach().to(torch.float32).contiguous()

        weights = (w_a_p, w_a_g, w_b_p, w_b_g)
        biases = (b_a_p, b_a_g, b_b_p, b_b_g)
        w_abpg = torch.cat([w.detach().to(torch.float32) for w in weights], 0).contiguous()
        b_abpg = None
        if any(b is not None for b in biases):
            b_abpg = torch.cat([torch.zeros(CHANNELS, device=w_abpg.device) if b is None
                                else b.detach().to(torch.float32).to(w_abpg.device)
                                for b in biases]).contiguous()
        return cls(prep(ln_in_w), prep(ln_in_b), w_abpg, b_abpg, prep(ln_out_w), prep(ln_out_b),
                   prep(w_z), prep(b_z), prep(w_g), prep(b_g), float(eps_in), float(eps_out))

    @classmethod
    def from_module(cls, module: Any) -> "TriMulWeights":
        """Protenix / OpenFold ``TriangleMultiplicativeUpdate``: ``layer_norm_in``,
        ``linear_{a,b}_{p,g}``, ``layer_norm_out``, ``linear_z``, ``linear_g``
        (triangle_multiplication.py:155-181)."""
        def bias(layer):
            return getattr(layer, "bias", None)
        return cls.from_tensors(
            ln_in_w=module.layer_norm_in.weight, ln_in_b=module.layer_norm_in.bias,
            w_a_p=module.linear_a_p.weight, w_a_g=module.linear_a_g.weight,
            w_b_p=module.linear_b_p.weight, w_b_g=module.linear_b_g.weight,
            ln_out_w=module.layer_norm_out.weight, ln_out_b=module.layer_norm_out.bias,
            w_z=module.linear_z.weight, w_g=module.linear_g.weight,
            b_a_p=bias(module.linear_a_p), b_a_g=bias(module.linear_a_g),
            b_b_p=bias(module.linear_b_p), b_b_g=bias(module.linear_b_g),
            b_z=bias(module.linear_z), b_g=bias(module.linear_g),
            eps_in=float(getattr(module.layer_norm_in, "eps", 1e-5)),
            eps_out=float(getattr(module.layer_norm_out, "eps", 1e-5)))

    def tensors(self) -> tuple[torch.Tensor | None, ...]:
        return (self.ln_in_w, self.ln_in_b, self.w_abpg, self.b_abpg, self.ln_out_w,
                self.ln_out_b, self.w_z, self.b_z, self.w_g, self.b_g)

    def to(self, device: Any) -> "TriMulWeights":
        moved = {f.name: getattr(self, f.name) for f in dataclasses.fields(self)}
        return TriMulWeights(**{k: (v.to(device) if isinstance(v, torch.Tensor) else v)
                                for k, v in moved.items()})


def workspace_bytes(n: int) -> int:
    size = _native.library().fpx_tri_mul_workspace_bytes(n, CHANNELS, CHANNELS)
    if size == 0:
        raise ValueError(f"unsupported triangle-multiplication size n={n}")
    return int(size)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def triangle_multiplication(z: torch.Tensor, mask: torch.Tensor | None, weights: TriMulWeights,
                            *, outgoing: bool, out: torch.Tensor | None = None,
                            accumulate: bool = False,
                            workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One ``fpx_tri_mul`` call on z's device and current stream.

    ``out`` defaults to a new ``[N, N, 128]`` tensor (the update); pass
    ``out=z`` for the in-place forms (``accumulate=True``: ``z += update``).
    """
    if not z.is_cuda or z.dtype != torch.float32:
        raise ValueError("z must be a float32 tensor on a HIP device")
    n = z.shape[0]
    if z.dim() != 3 or z.shape[1] != n or z.shape[2] != CHANNELS or z.stride(2) != 1:
        raise ValueError("z must be [N, N, 128] with unit channel stride")
    lib = _native.library()
    if out is None:
        out = torch.empty((n, n, CHANNELS), dtype=torch.float32, device=z.device)
    if tuple(out.shape) != tuple(z.shape) or out.stride(2) != 1 or out.dtype != torch.float32:
        raise ValueError("out must be float32 [N, N, 128] with unit channel stride")
    if mask is not None:
        if tuple(mask.shape) != (n, n):
            raise ValueError("mask must be [N, N]")
        if mask.dtype != torch.float32:
            mask = mask.to(torch.float32)
    size = workspace_bytes(n)
    if workspace is None:
        workspace = torch.empty(size, dtype=torch.uint8, device=z.device)
    w = weights
    with torch.cuda.device(z.device):
        code = lib.fpx_tri_mul(
            z.data_ptr(), z.stride(0), z.stride(1),
            _ptr(mask), mask.stride(0) if mask is not None else 0,
            mask.stride(1) if mask is not None else 0,
            _ptr(w.ln_in_w), _ptr(w.ln_in_b), w.eps_in, w.w_abpg.data_ptr(), _ptr(w.b_abpg),
            _ptr(w.ln_out_w), _ptr(w.ln_out_b), w.eps_out, w.w_z.data_ptr(), _ptr(w.b_z),
            w.w_g.data_ptr(), _ptr(w.b_g), n, CHANNELS, CHANNELS, int(bool(outgoing)),
            int(bool(accumulate)), out.data_ptr(), out.stride(0), out.stride(1),
            workspace.data_ptr(), workspace.numel(), torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_tri_mul")
    return out


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


def eligible(module: Any, z: Any, mask: Any) -> tuple[bool, str]:
    """The tensor/module contract that the signature cannot carry."""
    if not getattr(z, "is_cuda", False) or z.dtype != torch.float32:
        return False, "z is not a float32 HIP tensor"
    if (z.dim() != 3 or z.shape[0] != z.shape[1] or z.shape[2] != CHANNELS
            or not 1 <= z.shape[0] <= MAX_N):
        return False, "z must be [N, N, 128] with 1 <= N <= 4096"
    if z.stride(2) != 1 or z.stride(0) % 4 or z.stride(1) % 4 or z.data_ptr() % 16:
        return False, "z rows are not 16-byte aligned with unit channel stride"
    if mask is not None and (tuple(mask.shape) != tuple(z.shape[:2]) or mask.device != z.device):
        return False, "mask must be [N, N] on z's device"
    if getattr(module, "c_z", CHANNELS) != CHANNELS or getattr(module, "c_hidden",
                                                               CHANNELS) != CHANNELS:
        return False, "c_z and c_hidden must both be 128"
    try:
        layers = [getattr(module, name) for name in LINEARS]
        norms = [module.layer_norm_in, module.layer_norm_out]
    except AttributeError as error:
        return False, f"module layout: {error}"
    for layer in layers:
        weight = getattr(layer, "weight", None)
        if not isinstance(weight, torch.Tensor) or tuple(weight.shape) != (CHANNELS, CHANNELS):
            return False, "projection weights must be [128, 128] tensors"
    params = [getattr(layer, "weight", None) for layer in layers + norms]
    params += [getattr(layer, "bias", None) for layer in layers + norms]
    if any(t is not None and (t.device != z.device or not t.dtype.is_floating_point)
           for t in params):
        return False, "weights are not floating-point tensors on z's device"
    return True, ""


def _supports(signature: OperationSignature) -> bool | tuple[bool, str]:
    if (off := switches.rejection("FPX_DISABLE_TRIANGLE_MULTIPLICATION")) is not None:
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
    if attributes.get("c_z") != "128" or attributes.get("c_hidden") != "128":
        return False, "c_z and c_hidden must both be 128"
    if attributes.get("eligible") != "True":
        return False, attributes.get("reason", "tensor/module contract mismatch")
    if not _native.available():
        return False, "HIP extension unavailable"
    return True


def _hip(*, module: Any, z: Any, mask: Any, inplace_safe: bool, add_with_inplace: bool,
         inplace_chunk_size: int | None, native: Callable[..., Any]) -> Any:
    del inplace_chunk_size, native
    weights = TriMulWeights.from_module(module).to(z.device)
    outgoing = bool(module._outgoing)
    ws = ws_cache.get(z.device, workspace_bytes(z.shape[0]), purpose="triangle_multiplication")
    if inplace_safe:
        return triangle_multiplication(z, mask, weights, outgoing=outgoing, out=z,
                                       accumulate=add_with_inplace, workspace=ws)
    return triangle_multiplication(z, mask, weights, outgoing=outgoing, workspace=ws)


def dispatch_triangle_multiplication(*, module: Any, z: Any, mask: Any, inplace_safe: bool,
                                     add_with_inplace: bool, inplace_chunk_size: int | None,
                                     native: Callable[..., Any]) -> Any:
    """Select the HIP update or the caller's native function (same keyword
    contract and signature as the reference's dispatcher)."""
    mode = ("inference" if not getattr(module, "training", False) and not torch.is_grad_enabled()
            and not getattr(z, "requires_grad", False) else "training")
    ok, reason = eligible(module, z, mask)
    signature = signature_from_tensor(
        OPERATION, z, architecture=_architecture(z), mode=mode,
        mask="none" if mask is None else "dense", inplace=inplace_safe,
        attributes={"direction": "outgoing" if getattr(module, "_outgoing", True) else "incoming",
                    "add_with_inplace": add_with_inplace,
                    "c_z": getattr(module, "c_z", None), "c_hidden": getattr(module, "c_hidden", None),
                    "eligible": ok, "reason": reason})
    return registry.dispatch(signature, native, module=module, z=z, mask=mask,
                             inplace_safe=inplace_safe, add_with_inplace=add_with_inplace,
                             inplace_chunk_size=inplace_chunk_size, native=native)


registry.register(operation=OPERATION, name=IMPLEMENTATION, function=_hip, supports=_supports,
                  priority=40, version="1")
