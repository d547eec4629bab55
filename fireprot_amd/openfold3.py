"""OpenFold3 ``_attention`` served by the gfx950 attention core.

The reference swaps ``openfold3.core.model.primitives.attention._attention``
for a dispatcher inside an explicit scope (python/fireprot/adapters/openfold3/
attention.py:43-84) and keeps these rules, which callers rely on:

* the upstream source file must hash to a pinned SHA-256, and its
  ``_attention`` must still be the function defined in that file (the refusal
  messages "Unsupported OpenFold3 attention source" and "OpenFold3 attention
  was already replaced");
* one scope at a time, process-wide ("An OpenFold3 attention scope is already
  installed");
* only the execution context that opened the scope (and contexts copied from
  it while it is open) reaches the dispatcher; other threads keep calling the
  native function, and any reference to the installed callable that outlives
  the scope calls the native function too;
* on exit the native function is put back, unless someone replaced the
  installed callable meanwhile: then the foreign callable stays, the scope
  slot is released, and "OpenFold3 attention hook changed during its scope"
  is raised.

Here the installed callable is a ``ScopedAttentionHook`` object.  It is its
own context manager: entering claims the single process-wide slot, records the
native function, places itself on the module and marks itself active in a
context variable; a call checks that the active hook of the calling context
is this very object and that the scope is still open.

``AttentionDispatcher`` (attention.py:87-155) registers one candidate in a
private registry and routes eligible calls to it, everything else to the
native function.  The reference's fused candidate is still three steps: a QK
einsum, its mask+bias+softmax C ABI (backends/amd/softmax_fp32.py:57-84) over
the materialised ``[B, 4, N, N]`` scores, and a PV einsum.  Here the candidate
is ``StridedAttention``: one launch sequence of ``fpx_attn_strided`` that reads
q, k, v, the mask bias and the triangle bias in whatever strides the model
hands over (head-first, head-last and the transposed ending-node views),
stages them in the kernel's order and never writes the scores to memory.  Its
output is ``[B, 4, N, 32]`` viewed on ``[B, N, 4, 32]`` memory, so the model's
following ``transpose(-2, -3)`` and head flattening need no copy.

Both ``use_high_precision`` modes compute in FP32 (the reference runs both
under the same FP32 autocast context, attention.py:135-137).
"""
from __future__ import annotations

import hashlib
import threading
from contextlib import contextmanager
from contextvars import ContextVar
from pathlib import Path
from typing import Any

from . import _native, switches
from .registry import OperationRegistry, signature_from_tensor

# The upstream openfold3/core/model/primitives/attention.py the hook is written
# against (the same pin as attention.py:36): another source is refused.
SOURCE_SHA256 = "30fe5433982ee73e3d7ce5341fa6b510b1ea332dbde072d56129632cc53f0746"
OPERATION = "attention"
IMPLEMENTATION = "amd-gfx950-hip-attention-strided-f32"
VERSION = "strided-f32-v1"
ARCHITECTURE = "gfx950"
HEADS = 4
HEAD_DIM = 32
MAX_N = 4096

# The hook object active in the current execution context (threads start
# without one; copied contexts inherit it).
_active_hook: ContextVar[Any] = ContextVar("fireprot_amd_openfold3_active_hook", default=None)
# The hook that currently holds the process-wide scope (at most one).
_slot: list[Any] = []
_slot_guard = threading.Lock()


class ScopedAttentionHook:
    """The callable placed on ``module._attention`` for one scope, and the
    context manager that places and removes it.

    A call runs ``dispatcher(native, *args, **kwargs)`` when the calling
    context's active hook is this object and the scope is open; any other
    call (other threads, calls after the scope closed) runs ``native``.
    """

    def __init__(self, module: Any, dispatcher: Any):
        self.module = module
        self.dispatcher = dispatcher
        self.native: Any = None
        self.open = False
        self._token: Any = None

    def __call__(self, *args: Any, **kwargs: Any) -> Any:
        if self.open and _active_hook.get() is self:
            return self.dispatcher(self.native, *args, **kwargs)
        return self.native(*args, **kwargs)

    def __enter__(self) -> "ScopedAttentionHook":
        with _slot_guard:
            if _slot:
                raise RuntimeError("An OpenFold3 attention scope is already installed")
            self.native = self.module._attention
            _slot.append(self)
            self.open = True
            self.module._attention = self
            self._token = _active_hook.set(self)
        return self

    def __exit__(self, *exc_info: Any) -> bool:
        with _slot_guard:
            self.open = False
            _active_hook.reset(self._token)
            _slot.remove(self)
            displaced = self.module._attention is not self
            if not displaced:
                self.module._attention = self.native
        if displaced:
            raise RuntimeError("OpenFold3 attention hook changed during its scope")
        return False


def _verify_upstream(module: Any) -> None:
    """The pinned source file, and its own ``_attention`` still in place."""
    source = Path(module.__file__).resolve()
    if hashlib.sha256(source.read_bytes()).hexdigest() != SOURCE_SHA256:
        raise RuntimeError("Unsupported OpenFold3 attention source")
    code = getattr(module._attention, "__code__", None)
    defined_here = (code is not None and code.co_name == "_attention"
                    and Path(code.co_filename).resolve() == source)
    if not defined_here:
        raise RuntimeError("OpenFold3 attention was already replaced")


@contextmanager
def attention_scope(dispatcher: Any, module: Any = None):
    """Scope in which OpenFold3's ``_attention`` goes through ``dispatcher``
    (called as ``dispatcher(native, *args, **kwargs)``).

    ``module`` defaults to ``openfold3.core.model.primitives.attention``; its
    source must hash to ``SOURCE_SHA256`` and its ``_attention`` must be the
    function defined there.  Yields the installed hook.
    """
    if module is None:
        import openfold3.core.model.primitives.attention as module  # noqa: PLC0415
    _verify_upstream(module)
    with ScopedAttentionHook(module, dispatcher) as hook:
        yield hook


def _architecture(index: int) -> str:
    import torch

    return str(getattr(torch.cuda.get_device_properties(index), "gcnArchName", "")).split(":")[0]


def tensor_contract(query: Any, key: Any, value: Any, biases: Any) -> tuple[bool, str]:
    """The tensor contract of one fused launch (no device or library checks).

    q, k, v ``[B, 4, N, 32]`` float32 with ``1 <= N <= 4096``; biases exactly
    ``[mask_bias [B|1, 1, 1, N], triangle_bias [1, 4, N, N]]`` float32 on the
    same device; no autograd, negative strides, or neg/conj views
    (attention.py:99-119 and softmax_fp32.py:19-38, without their N in
    {1000, 1536} and B <= 1536 limits, which came from the published kernel).
    """
    import torch

    if torch.is_grad_enabled():
        return False, "autograd is enabled"
    if not isinstance(biases, (tuple, list)) or len(biases) != 2:
        return False, "biases must be [mask_bias, triangle_bias]"
    tensors = (query, key, value, *biases)
    if any(type(t) is not torch.Tensor for t in tensors):
        return False, "arguments must be plain tensors"
    if any(t.dtype != torch.float32 or not t.is_cuda or t.device != query.device
           or t.requires_grad or t.is_neg() or t.is_conj() for t in tensors):
        return False, "tensors must be float32 on one HIP device without autograd"
    if query.ndim != 4 or key.shape != query.shape or value.shape != query.shape:
        return False, "q, k, v must be [B, H, N, D] of one shape"
    batch, heads, n, dim = query.shape
    if heads != HEADS or dim != HEAD_DIM or not 1 <= n <= MAX_N or batch < 1:
        return False, "requires 4 heads of dimension 32 and 1 <= N <= 4096"
    mask, bias = biases
    if (mask.ndim != 4 or mask.shape[0] not in (1, batch) or tuple(mask.shape[1:]) != (1, 1, n)
            or tuple(bias.shape) != (1, HEADS, n, n)):
        return False, "biases must be [B|1, 1, 1, N] and [1, 4, N, N]"
    if any(s < 0 for t in tensors for s in t.stride()):
        return False, "negative strides"
    return True, ""


def _operand(t: Any) -> Any:
    """``t`` itself when the kernel reads its layout (channel stride 1, 16-byte
    rows and base, a (b, h) slice below 2 GiB), else a contiguous copy."""
    s = t.stride()
    slice_bytes = ((t.shape[2] - 1) * s[2] + HEAD_DIM) * 4
    if (s[3] == 1 and all(x % 4 == 0 for x in s[:3]) and t.data_ptr() % 16 == 0
            and slice_bytes < 2 ** 31 - 1):
        return t
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class StridedAttention:
    """Fused ``_attention(q, k, v, [mask_bias, tri_bias])`` on gfx950.

    Plays the role of the reference's ``SoftmaxFP32`` kernel object
    (softmax_fp32.py:41-84): bound to one device, ``supports`` checks a call,
    ``__call__`` launches on the current stream and raises on a nonzero status.
    Construction fails loudly without a gfx950 device or the native library.
    """

    def __init__(self, device: int | None = None):
        import torch

        if not torch.cuda.is_available():
            raise RuntimeError("HIP GPU unavailable")
        index = torch.cuda.current_device() if device is None else int(device)
        if _architecture(index) != ARCHITECTURE:
            raise RuntimeError(f"strided attention requires {ARCHITECTURE}")
        self.library = _native.library()
        self.device = index
        self.launches_submitted = 0
        self.receipt = {"library": str(_native.LIB_PATH), "abi": self.library.fpx_abi_version(),
                        "entry": "fpx_attn_strided", "version": VERSION}

    def supports(self, query: Any, key: Any, value: Any, biases: Any) -> bool:
        ok, _ = tensor_contract(query, key, value, biases)
        return ok and query.device.index == self.device

    def __call__(self, query: Any, key: Any, value: Any, biases: Any,
                 workspace: Any = None) -> Any:
        """``workspace``: an optional uint8 device tensor of at least
        ``fpx_attn_strided_workspace_bytes(B, N)`` bytes (any contents; a
        fresh one is allocated when omitted)."""
        import torch

        if not self.supports(query, key, value, biases):
            raise ValueError("Unsupported attention tensors or device")
        mask, bias = biases
        batch, _, n, _ = query.shape
        q, k, v = _operand(query), _operand(key), _operand(value)
        with torch.cuda.device(self.device):
            out = torch.empty((batch, n, HEADS, HEAD_DIM), device=query.device,
                              dtype=torch.float32).transpose(1, 2)
            size = self.library.fpx_attn_strided_workspace_bytes(batch, n)
            if workspace is None:
                workspace = torch.empty(size, dtype=torch.uint8, device=query.device)
            elif (workspace.dtype != torch.uint8 or workspace.device != query.device
                  or workspace.numel() < size):
                raise ValueError(f"workspace needs {size} bytes on {query.device}")
            code = self.library.fpx_attn_strided(
                q.data_ptr(), *q.stride()[:3], k.data_ptr(), *k.stride()[:3],
                v.data_ptr(), *v.stride()[:3],
                mask.data_ptr(), mask.stride(0) if mask.shape[0] > 1 else 0, mask.stride(3),
                bias.data_ptr(), *bias.stride()[1:],
                out.data_ptr(), *out.stride()[:3], batch, n,
                workspace.data_ptr(), size, torch.cuda.current_stream().cuda_stream)
        _native.check(code, "fpx_attn_strided")
        self.launches_submitted += 1
        return out


class AttentionDispatcher:
    """Route OpenFold3 ``_attention`` calls: eligible ones to ``kernel`` (a
    ``StridedAttention``, or ``None`` for native-only dispatch), the rest to
    the native function the hook captured (attention.py:87-133)."""

    def __init__(self, kernel: StridedAttention | None):
        self.kernel = kernel
        self.registry = OperationRegistry()
        self.registry.register(
            operation=OPERATION, name=IMPLEMENTATION, function=self._fused, priority=10,
            version=VERSION, supports=self._supports)

    @staticmethod
    def _supports(signature: Any) -> tuple[bool, str]:
        attributes = dict(signature.attributes)
        if attributes.get("eligible") == "True":
            return True, ""
        return False, attributes.get("reason") or "tensor contract mismatch"

    def _eligible(self, query: Any, key: Any, value: Any, biases: Any) -> tuple[bool, str]:
        if (off := switches.rejection("FPX_DISABLE_OPENFOLD3_ATTENTION")) is not None:
            return off
        if self.kernel is None:
            return False, "no HIP kernel"
        ok, reason = tensor_contract(query, key, value, biases)
        if ok and query.device.index != self.kernel.device:
            return False, "tensors are not on the kernel's device"
        return ok, reason

    def __call__(self, native: Any, query: Any, key: Any, value: Any, biases: Any,
                 use_high_precision: bool = False) -> Any:
        import torch

        if type(query) is not torch.Tensor:
            return native(query, key, value, biases, use_high_precision=use_high_precision)
        eligible, reason = self._eligible(query, key, value, biases)
        signature = signature_from_tensor(
            OPERATION, query,
            architecture=ARCHITECTURE if self.kernel is not None else "unknown",
            mode="training" if torch.is_grad_enabled() else "inference",
            mask="pair_and_token", inplace=False,
            attributes={"eligible": eligible, "reason": reason,
                        "high_precision": use_high_precision})
        return self.registry.dispatch(signature, native, query, key, value, biases,
                                      use_high_precision=use_high_precision)

    def _fused(self, query: Any, key: Any, value: Any, biases: Any,
               use_high_precision: bool = False) -> Any:
        del use_high_precision  # FP32 logits, weights and accumulation either way
        return self.kernel(query, key, value, biases)

    def manifest(self) -> dict[str, Any]:
        return {
            "registry": self.registry.manifest(),
            "kernel": None if self.kernel is None else self.kernel.receipt,
            "launches_submitted": 0 if self.kernel is None else self.kernel.launches_submitted,
        }
