"""Capability-gated triangle-attention dispatch on gfx950.

Two operations are registered in the shared ``fireprot_amd.registry``:

``triangle_attention`` -- the attention core behind Protenix
``Attention.forward``'s ``triangle_attention="fireprot"`` branch
(patches/protenix/0002-*.patch:46-58).  ``dispatch_triangle_attention`` has the
reference's signature and builds the same ``OperationSignature``
(python/fireprot/backends/amd/triangle_attention.py:199-256); the HIP
candidate ``amd-gfx950-hip-attention-f32`` takes q/k/v ``[B, H, N, 32]`` in
the head-last projection layout (strides ``(N*128, 32, 128, 1)``), the
triangle bias ``[1, 4, N, N]`` (any strides) and optionally the mask bias
``[B|1, 1, 1, N]``, and returns ``[B, N, H, 32]`` like the native lambda
``_attention(q, k, v, biases).transpose(-2, -3)``.  It runs
``fpx_attn_strided`` (q, k, v staged into power-of-two scaled fp16 planes,
then the block's attention kernel on the 16-bit matrix cores, FP32-accurate)
with a workspace cached per device and stream; the reference's workspace-less
entries ``ck_attention*`` stay on the FP32 matrix cores.

``triangle_attention_block`` -- the whole module call ``(z, mask) -> dz``,
as AtlasFold's per-instance hook dispatches it
(python/fireprot/adapters/atlasfold/runtime.py:185-207).  The module's
weights are read through ``BlockWeights.from_protenix`` or
``from_atlasfold``.

Unsupported calls go to the caller's ``native`` function, never to a CPU
path of this package.
"""
from __future__ import annotations

import functools
import math
import weakref
from collections.abc import Callable, Sequence
from typing import Any

from . import _native, switches
from . import workspace as ws_cache
from .block import BlockWeights, triangle_attention_block, workspace_bytes
from .registry import OperationSignature, registry, signature_from_tensor

OPERATION = "triangle_attention"
BLOCK_OPERATION = "triangle_attention_block"
IMPLEMENTATION = "amd-gfx950-hip-attention-f32"
BLOCK_IMPLEMENTATION = "amd-gfx950-hip-block-f32"
BLOCK_BF16_IMPLEMENTATION = "amd-gfx950-hip-block-bf16"
ARCHITECTURE = "gfx950"
HEADS = 4
HEAD_DIM = 32
MAX_N = 4096  # the largest pair size the block and strided C ABI entries accept


@functools.lru_cache(maxsize=None)
def _device_architecture(index: int) -> str:
    import torch

    properties = torch.cuda.get_device_properties(index)
    return str(getattr(properties, "gcnArchName", "")).split(":", 1)[0]


def _architecture(tensor: Any) -> str:
    try:
        if tensor.device.type != "cuda":
            return "cpu"
        return _device_architecture(int(tensor.device.index or 0))
    except Exception:
        return "unknown"


def _mode(module: Any, tensors: Sequence[Any]) -> str:
    import torch

    training = bool(getattr(module, "training", False))
    if not training and not torch.is_grad_enabled() and not any(t.requires_grad for t in tensors):
        return "inference"
    return "training"


# ------------------------------------------------------------------ core

def _supports_core(signature: OperationSignature) -> bool | tuple[bool, str]:
    if (off := switches.rejection("FPX_DISABLE_ATTENTION")) is not None:
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
    if len(signature.shape) != 4:
        return False, "q must be [B, H, N, D]"
    batch, heads, n, dim = signature.shape
    if heads != HEADS or dim != HEAD_DIM:
        return False, "requires 4 heads of dimension 32"
    if not 1 <= n <= MAX_N:
        return False, f"sequence length must lie in 1..{MAX_N}"
    strides = (n * HEADS * HEAD_DIM, HEAD_DIM, HEADS * HEAD_DIM, 1)
    if attributes.get("qkv_strides") != repr((strides,) * 3):
        return False, "q/k/v must use the head-last projection layout"
    shapes = attributes.get("bias_shapes")
    allowed = {repr(((1, HEADS, n, n),)),
               repr(((batch, 1, 1, n), (1, HEADS, n, n))),
               repr(((1, 1, 1, n), (1, HEADS, n, n)))}
    if shapes not in allowed:
        return False, "biases must be [mask_bias [B|1,1,1,N],] triangle bias [1,4,N,N]"
    if attributes.get("ck_tile_compatible") != "True":
        return False, "q/k/v/bias dtype, device or 16-byte alignment mismatch"
    if not _native.available():
        return False, "HIP extension unavailable"
    return True


def attention(*, module: Any, q: Any, k: Any, v: Any, biases: Sequence[Any],
              native: Callable[..., Any]) -> Any:
    """HIP flash attention; returns ``[B, N, H, D]`` (contiguous)."""
    import torch

    del module, native
    lib = _native.library()
    batch, _, n, _ = q.shape
    bias = biases[-1]
    if bias.data_ptr() % 4:
        bias = bias.contiguous()
    mask_ptr, m_sb, m_sk = None, 0, 0
    if len(biases) == 2:
        mask = biases[0]
        if mask.data_ptr() % 4:
            mask = mask.contiguous()
        mask_ptr = mask.data_ptr()
        m_sb = mask.stride(0) if mask.shape[0] > 1 else 0
        m_sk = mask.stride(3)
    with torch.cuda.device(q.device):
        output = torch.empty((batch, n, HEADS, HEAD_DIM), device=q.device, dtype=q.dtype)
        size = lib.fpx_attn_strided_workspace_bytes(batch, n)
        ws = ws_cache.get(q.device, size, purpose="attention")
        o = output.transpose(1, 2)  # [B, H, N, D] view of the head-last output
        code = lib.fpx_attn_strided(
            q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
            v.data_ptr(), *v.stride()[:3], mask_ptr, m_sb, m_sk,
            bias.data_ptr(), *bias.stride()[1:], o.data_ptr(), *o.stride()[:3], batch, n,
            ws.data_ptr(), size, torch.cuda.current_stream(q.device).cuda_stream)
    _native.check(code, "fpx_attn_strided")
    return output


def dispatch_triangle_attention(*, module: Any, q: Any, k: Any, v: Any, biases: Sequence[Any],
                                native: Callable[..., Any]) -> Any:
    """Select the HIP core or the caller's native lambda (same contract as the
    reference's ``dispatch_triangle_attention``)."""
    bias_shapes = tuple(tuple(int(x) for x in b.shape) for b in biases)
    signature = signature_from_tensor(
        OPERATION, q, architecture=_architecture(q), mode=_mode(module, (q, k, v)),
        mask=("triangle-bias" if len(biases) == 1
              else "additive-mask-and-triangle-bias" if len(biases) == 2 else "unsupported"),
        inplace=False,
        attributes={
            "bias_count": len(biases),
            "bias_shapes": repr(bias_shapes),
            "qkv_strides": repr(tuple(tuple(t.stride()) for t in (q, k, v))),
            "ck_tile_compatible": (
                all(t.shape == q.shape and t.dtype == q.dtype and t.device == q.device
                    and t.data_ptr() % 16 == 0 for t in (q, k, v))
                and all(b.dtype == q.dtype and b.device == q.device for b in biases)),
            "heads": q.shape[-3] if q.ndim >= 3 else -1,
            "head_dim": q.shape[-1] if q.ndim else -1,
        })
    return registry.dispatch(signature, native, module=module, q=q, k=k, v=v, biases=biases,
                             native=native)


# ----------------------------------------------------------------- block


# Packed weights per module, rebuilt only when one of the module's parameter
# tensors changes (identity, storage or in-place version) or the device does.
_packed: "weakref.WeakKeyDictionary[Any, tuple[tuple, BlockWeights]]" = weakref.WeakKeyDictionary()


def _layers(module: Any) -> tuple[tuple, tuple]:
    """The layers whose weights the block packs, in packing order, and the
    other sub-layers whose hooks would run in the module's own forward
    (Protenix: patches/protenix/0005-*.patch:32-45; AtlasFold:
    python/fireprot/adapters/atlasfold/runtime.py:224-233)."""
    if hasattr(module, "mha"):
        mha = module.mha
        return ((module.layer_norm, module.linear, mha.linear_q, mha.linear_k, mha.linear_v,
                 mha.linear_g, mha.linear_o), (mha,))
    if hasattr(module, "linear_qkv"):
        return ((module.layernorm, module.linear_qkv, module.linear_bias, module.linear_g,
                 module.linear_out), ())
    raise TypeError(f"unrecognised triangle-attention module {type(module).__name__}")


def _tensor(owner: Any, name: str) -> Any:
    """``owner.<name>`` or None; a registered parameter is read from the
    module's parameter table (``nn.Module`` attribute lookup would go through
    its Python ``__getattr__``)."""
    params = getattr(owner, "__dict__", {}).get("_parameters")
    if params is not None and name in params:
        return params[name]
    return getattr(owner, name, None)


def _parameter_key(module: Any, layers: tuple | None = None) -> tuple | None:
    """Identity, storage and version of every tensor _weights_of reads, or
    None when one of them is an inference tensor (created under
    ``torch.inference_mode``: such tensors keep no version counter, so an
    in-place change could not be seen and the weights are packed afresh)."""
    key = []
    for owner in (_layers(module)[0] if layers is None else layers):
        for name in ("weight", "bias"):
            t = _tensor(owner, name)
            if t is None:
                key.append(None)
                continue
            if t.is_inference():
                return None
            key.append((id(t), t.data_ptr(), t._version, t.dtype, t.device))
    key.append(float(getattr(module, "inf", 1e9)))
    return tuple(key)


def _pack_dtype(z: Any) -> Any:
    """z's dtype when a CUDA autocast region computes in it (the module's
    linears would then run on weights cast to it), else None: keep the
    weights' own dtype."""
    import torch

    try:
        if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == z.dtype:
            return z.dtype
    except (AttributeError, TypeError):
        pass
    return None


def _weights_of(module: Any, dtype: Any = None, layers: tuple | None = None) -> BlockWeights:
    """The module's weights packed for the block (w_qkvg concatenated) in
    ``dtype`` (default: the weights' own), cached per module while its
    parameters are unchanged."""
    if layers is None:
        layers = _layers(module)[0]
    try:
        key = _parameter_key(module, layers)
        key = None if key is None else key + (str(dtype),)
        hit = None if key is None else _packed.get(module)
    except TypeError:  # not weak-referenceable: no cache
        key, hit = None, None
    if hit is not None and hit[0] == key:
        return hit[1]
    weights = (BlockWeights.from_protenix(module, dtype=dtype) if hasattr(module, "mha")
               else BlockWeights.from_atlasfold(module, dtype=dtype))
    if key is not None:
        try:
            _packed[module] = (key, weights)
        except TypeError:
            pass
    return weights


def _precision(layer: Any) -> Any:
    """The layer's ``precision`` override, or None.  When its class defines
    no ``precision`` (a value or a property), the instance dictionary holds
    it or nothing does; reading it there spares ``nn.Module.__getattr__`` the
    exception of a missing attribute."""
    if hasattr(type(layer), "precision"):
        return getattr(layer, "precision", None)
    return getattr(layer, "__dict__", {}).get("precision")


def _has_hooks(module: Any, layers: tuple[tuple, tuple] | None = None) -> bool:
    """Forward hooks on the module or the layers the block reads, or a
    ``precision`` override on them: the fused block would skip them
    (atlasfold/runtime.py:224-233 rejects the same)."""
    import torch

    packed, others = _layers(module) if layers is None else layers
    for layer in (module, *others, *packed):
        if isinstance(layer, torch.nn.Module) and (layer._forward_hooks or
                                                   layer._forward_pre_hooks):
            return True
        if layer is not module and _precision(layer) is not None:
            return True
    return False


def _block_check(module: Any, z: Any, mask: Any) -> tuple[bool, str, BlockWeights | None]:
    """block_eligible's verdict and, when it passes, the packed weights."""
    import torch

    if not getattr(z, "is_cuda", False) or z.dtype not in (torch.float32, torch.bfloat16):
        return False, "z is not a float32 or bfloat16 HIP tensor", None
    if z.dim() != 3 or z.shape[0] != z.shape[1] or z.shape[2] != 128 or z.stride(2) != 1:
        return False, "z must be [N, N, 128] with unit channel stride", None
    if not 1 <= z.shape[0] <= MAX_N:
        return False, f"N must lie in 1..{MAX_N}", None
    align = 16 // z.element_size()
    if z.stride(0) % align or z.stride(1) % align or z.data_ptr() % 16:
        return False, "z rows are not 16-byte aligned", None
    if mask is not None and (tuple(mask.shape) != tuple(z.shape[:2]) or mask.device != z.device):
        return False, "mask must be [N, N] on z's device", None
    owner = getattr(module, "mha", module)
    heads = getattr(owner, "no_heads", None)
    if heads is None:
        heads = getattr(module, "num_heads", None)
    dim = getattr(owner, "c_hidden", None)
    if dim is None:
        dim = getattr(module, "channel_hidden", None)
    if heads != HEADS or dim != HEAD_DIM:
        return False, "module must have 4 heads of dimension 32", None
    scale = getattr(module, "scale", None)
    if scale is not None and abs(float(scale) * math.sqrt(HEAD_DIM) - 1.0) > 1e-6:
        return False, "module q scale is not 1/sqrt(32)", None
    try:
        layers = _layers(module)
        if _has_hooks(module, layers):
            return (False, "module or one of its layers carries forward hooks or a precision "
                    "override", None)
        weights = _weights_of(module, _pack_dtype(z), layers[0])
    except (AttributeError, TypeError, ValueError, RuntimeError) as error:
        return False, f"module layout: {error}", None
    if any(t is not None and (t.device != z.device or t.dtype != z.dtype)
           for t in weights.tensors()):
        return False, "weights do not have z's dtype and device", None
    return True, "", weights


def block_eligible(module: Any, z: Any, mask: Any) -> tuple[bool, str]:
    """Check the tensor/module contract that the signature cannot carry."""
    eligible, reason, _ = _block_check(module, z, mask)
    return eligible, reason


def _supports_block(signature: OperationSignature, *,
                    dtype: str = "float32") -> bool | tuple[bool, str]:
    flag = "FPX_DISABLE_BLOCK" if dtype == "float32" else "FPX_DISABLE_BLOCK_BF16"
    if (off := switches.rejection(flag)) is not None:
        return off
    attributes = dict(signature.attributes)
    if signature.device_type != "cuda":
        return False, "device is not CUDA/HIP"
    if signature.architecture != ARCHITECTURE:
        return False, f"architecture is not {ARCHITECTURE}"
    if signature.dtype != dtype:
        return False, f"dtype is not {dtype}"
    if signature.mode != "inference":
        return False, "training or autograd is enabled"
    if attributes.get("eligible") != "True":
        return False, attributes.get("reason", "tensor/module contract mismatch")
    if not _native.available():
        return False, "HIP extension unavailable"
    return True


def _run_block(z: Any, mask: Any, weights: BlockWeights, ending: bool) -> Any:
    """One block call with the workspace cached for z's device and stream."""
    ws = ws_cache.get(z.device, workspace_bytes(z.shape[0], z.dtype), purpose="block")
    return triangle_attention_block(z, mask, weights, ending=ending, workspace=ws)


def _block(*, module: Any, z: Any, mask: Any, ending: bool, native: Any) -> Any:
    """The registered implementation: the module's packed weights, then one
    block call (the weights' device and dtype are checked again there)."""
    del native
    return _run_block(z, mask, _weights_of(module, _pack_dtype(z)), ending)


def dispatch_triangle_attention_block(*, module: Any, z: Any, mask: Any, ending: bool,
                                      native: Callable[..., Any]) -> Any:
    """Module-level drop-in ``(z, mask) -> dz`` with native fallback.

    The registry selects as ``registry.dispatch`` does; when it selects one of
    this module's block candidates, the weights the eligibility check packed
    are used directly (one walk over the module per call)."""
    eligible, reason, weights = _block_check(module, z, mask)
    signature = signature_from_tensor(
        BLOCK_OPERATION, z, architecture=_architecture(z),
        mode=_mode(module, (z,)), mask="none" if mask is None else "pair-mask", inplace=False,
        attributes={"eligible": eligible, "reason": reason, "ending": bool(ending)})
    chosen = registry.resolve(signature).implementation
    if chosen is not None and chosen.function is _block and weights is not None:
        return _run_block(z, mask, weights, ending)
    function = chosen.function if chosen is not None else native
    return function(module=module, z=z, mask=mask, ending=ending, native=native)


registry.register(operation=OPERATION, name=IMPLEMENTATION, function=attention,
                  supports=_supports_core, priority=30, version="1")
registry.register(operation=BLOCK_OPERATION, name=BLOCK_IMPLEMENTATION, function=_block,
                  supports=_supports_block, priority=30, version="1")
registry.register(operation=BLOCK_OPERATION, name=BLOCK_BF16_IMPLEMENTATION, function=_block,
                  supports=lambda signature: _supports_block(signature, dtype="bfloat16"),
                  priority=30, version="1")
