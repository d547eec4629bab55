"""View-based pair transpose around the ending node.

``transpose_pair(x, training=)`` mirrors the reference hook
(python/fireprot/backends/amd/pair_layout.py:8-26; call sites in
patches/protenix/0006-*.patch:17-37): when the next consumer reads through
strides it returns the ``x.transpose(-2, -3)`` view with no copy, otherwise the
contiguous transpose.  The gfx950 block and LayerNorm both read strided rows,
so every float32 inference square pair tensor on a gfx950 device qualifies.
"""
from __future__ import annotations

from typing import Any

from . import _native
from .triangle_attention import ARCHITECTURE, _architecture


def transpose_pair(x: Any, *, training: bool) -> Any:
    import torch

    view = x.transpose(-2, -3)
    supported = (not training and not torch.is_grad_enabled() and getattr(x, "is_cuda", False)
                 and x.dtype == torch.float32 and not x.requires_grad and x.dim() == 3
                 and x.shape[0] == x.shape[1] and x.shape[2] == 128 and x.stride(2) == 1
                 and x.data_ptr() % 16 == 0 and _architecture(x) == ARCHITECTURE
                 and _native.available())
    return view if supported else view.contiguous()
