"""Install the module-level drop-in into Protenix and AtlasFold models.

Both entry points route a triangle-attention module call ``(z, mask) -> dz``
through ``triangle_attention.dispatch_triangle_attention_block``: the
registry picks the HIP block when the call fits its contract and falls back to
the module's own forward otherwise.  The residual ``z += dz`` stays with the
caller (patches/protenix/0006-*.patch:25).

``install_protenix`` replaces ``TriangleAttention.forward`` on the class
before or after model construction, the way the reference's Protenix hooks
replace class methods with ``functools.wraps`` wrappers
(python/fireprot/adapters/protenix/hooks.py:26-140): idempotent, guarded by a
lock, reversible with ``uninstall_protenix``.  ``AtlasFoldHooks`` replaces
``forward`` per module instance, as the reference's AtlasFold runtime does
(python/fireprot/adapters/atlasfold/runtime.py:92-159), and puts the original
bound methods back on ``uninstall``.

Both refuse to stack on code they do not know (runtime.py:140-157): a
forward that is already a wrapper (``__wrapped__``) or already replaced on an
instance, a class method whose code lives outside the class's own source
file, or a model that already carries these hooks.  Neither upstream package
is importable here, so the classes can be passed in; by default they are
imported from their upstream modules.
"""
from __future__ import annotations

import functools
import inspect
import threading
import types
from typing import Any

import torch

from . import triangle_attention as ta

_lock = threading.RLock()
_protenix: dict[str, Any] = {"installed": False, "cls": None, "original": None}


def _check_class_forward(cls: type) -> None:
    """Refuse a forward that is already wrapped or was replaced from outside
    the class's own source file."""
    forward = cls.__dict__.get("forward", getattr(cls, "forward", None))
    if forward is None:
        raise ValueError(f"{cls.__name__} has no forward")
    if hasattr(forward, "__wrapped__"):
        raise ValueError("Refusing an already modified triangle forward")
    code = getattr(forward, "__code__", None)
    try:
        home = inspect.getsourcefile(cls)
    except TypeError:
        home = None
    if code is None or home is None or code.co_filename != home:
        raise ValueError("Refusing a replaced triangle class method")


def _squeeze(z: Any, mask: Any) -> tuple[Any, Any, bool]:
    """z ``[N, N, C]`` or ``[1, N, N, C]`` (mask ``[N, N]`` or ``[1, N, N]``)
    -> the 3-D form the block takes; boolean masks as float {0, 1}."""
    batched = isinstance(z, torch.Tensor) and z.dim() == 4 and z.shape[0] == 1
    if batched:
        z = z[0]
        if mask is not None and mask.dim() == 3 and mask.shape[0] == 1:
            mask = mask[0]
    if isinstance(mask, torch.Tensor) and mask.dtype == torch.bool:
        mask = mask.to(torch.float32)
    return z, mask, batched


# ---------------------------------------------------------------- Protenix

def install_protenix(triangle_attention_cls: type | None = None) -> dict[str, Any]:
    """Route ``TriangleAttention.forward(x, mask=None, ...)`` through the block
    dispatch (``ending = not self.starting``).  Calls the block cannot serve
    (training, autograd, other shapes or dtypes, a CPU tensor, a disabled
    path) run the original forward with the same arguments."""
    with _lock:
        if _protenix["installed"]:
            if triangle_attention_cls not in (None, _protenix["cls"]):
                raise ValueError("install_protenix is already installed on another class")
            return protenix_manifest()
        if triangle_attention_cls is None:
            from protenix.model.triangular.triangular import TriangleAttention  # noqa: PLC0415

            triangle_attention_cls = TriangleAttention
        cls = triangle_attention_cls
        _check_class_forward(cls)
        original = cls.forward

        @functools.wraps(original)
        def forward(self: Any, x: Any, mask: Any = None, *args: Any, **kwargs: Any) -> Any:
            def native(**_: Any) -> Any:
                return original(self, x, mask, *args, **kwargs)

            z, m, batched = _squeeze(x, mask)
            dz = ta.dispatch_triangle_attention_block(
                module=self, z=z, mask=m, ending=not bool(getattr(self, "starting", True)),
                native=native)
            return dz.unsqueeze(0) if batched and dz.dim() == 3 else dz

        forward.__fpx_hook__ = True
        cls.forward = forward
        _protenix.update(installed=True, cls=cls, original=original)
        return protenix_manifest()


def uninstall_protenix() -> dict[str, Any]:
    """Put the original ``TriangleAttention.forward`` back (no-op when not
    installed; refuses when someone replaced the hook since)."""
    with _lock:
        if not _protenix["installed"]:
            return protenix_manifest()
        cls = _protenix["cls"]
        if not getattr(cls.__dict__.get("forward"), "__fpx_hook__", False):
            raise ValueError("TriangleAttention.forward was replaced after install_protenix")
        cls.forward = _protenix["original"]
        _protenix.update(installed=False, cls=None, original=None)
        return protenix_manifest()


def protenix_manifest() -> dict[str, Any]:
    with _lock:
        cls = _protenix["cls"]
        return {"installed": _protenix["installed"],
                "hooks": [f"{cls.__name__}.forward"] if cls is not None else [],
                "registry": ta.registry.manifest()}


# ---------------------------------------------------------------- AtlasFold

class AtlasFoldHooks:
    """Per-instance ``forward(z, mask, kernel_backend='torch')`` replacement on
    every starting- and ending-node triangle-attention module of ``model``.

    ``starting_cls`` / ``ending_cls`` default to AtlasFold's
    ``TriangleAttentionStartingNode`` / ``TriangleAttentionEndingNode``.  A
    call with ``kernel_backend != 'torch'`` keeps its original forward, as do
    calls the block cannot serve.  z ``[1, N, N, 128]`` with a boolean mask
    ``[1, N, N]`` (AtlasFold's monomer form) or unbatched ``[N, N, 128]``.
    """

    ATTRIBUTE = "_fpx_atlasfold_hooks"

    def __init__(self, model: Any, *, starting_cls: type | None = None,
                 ending_cls: type | None = None):
        if starting_cls is None or ending_cls is None:
            from atlasfold.model.network.primitives.triangle_update import (  # noqa: PLC0415
                TriangleAttentionEndingNode, TriangleAttentionStartingNode)

            starting_cls = starting_cls or TriangleAttentionStartingNode
            ending_cls = ending_cls or TriangleAttentionEndingNode
        if getattr(model, "training", False):
            raise ValueError("Expected a model in eval mode")
        if getattr(model, self.ATTRIBUTE, None) is not None:
            raise ValueError("fireprot_amd AtlasFold hooks are already installed")
        types_to_hook = {starting_cls: False, ending_cls: True}
        modules = [m for m in model.modules() if type(m) in types_to_hook]
        for module in modules:  # refuse before changing anything
            if "forward" in module.__dict__ or hasattr(type(module).forward, "__wrapped__"):
                raise ValueError("Refusing an already modified triangle forward")
            _check_class_forward(type(module))
        self.originals: list[tuple[Any, Any]] = []
        self.counts = {"dispatched": 0, "kept": 0}
        for module in modules:
            original = module.forward
            ending = types_to_hook[type(module)]

            def forward(current: Any, z: Any, mask: Any, kernel_backend: str = "torch",
                        _original: Any = original, _ending: bool = ending) -> Any:
                return self._dispatch(current, z, mask, kernel_backend, _original, _ending)

            module.forward = types.MethodType(forward, module)
            self.originals.append((module, original))
        self.model = model
        setattr(model, self.ATTRIBUTE, self)

    def _dispatch(self, module: Any, z: Any, mask: Any, kernel_backend: str, original: Any,
                  ending: bool) -> Any:
        def native(**_: Any) -> Any:
            return original(z, mask, kernel_backend)

        if kernel_backend != "torch":
            self.counts["kept"] += 1
            return native()
        self.counts["dispatched"] += 1
        z3, m, batched = _squeeze(z, mask)
        dz = ta.dispatch_triangle_attention_block(module=module, z=z3, mask=m, ending=ending,
                                                  native=native)
        return dz.unsqueeze(0) if batched and dz.dim() == 3 else dz

    def uninstall(self) -> None:
        """Remove the instance forwards (the class method shows through again)."""
        for module, _ in self.originals:
            module.__dict__.pop("forward", None)
        self.originals = []
        if getattr(self.model, self.ATTRIBUTE, None) is self:
            delattr(self.model, self.ATTRIBUTE)
