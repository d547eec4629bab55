"""Cached device workspaces for the registered (module- and operator-level)
routes.

The C ABI entries never allocate: the caller passes a workspace of at least
the entry's ``*_workspace_bytes(...)``.  The registered candidates are called
per module call, so they keep one uint8 buffer per (device, stream) and grow
it when a call needs more, instead of asking the caching allocator for a
multi-GB block on every call (6.2 GB for a block at N=1536).

Keying by stream keeps two streams of one device from sharing a buffer
(their calls may overlap); calls on one stream are ordered, so they can
share.  Each buffer is allocated while its stream is current, so when a
smaller one is dropped for a larger one, the caching allocator reuses its
memory only for work queued later on that same stream.  ``release()`` drops
every cached buffer.
"""
from __future__ import annotations

import threading
from typing import Any

_lock = threading.Lock()
_buffers: dict[tuple[int, int, str], Any] = {}


def get(device: Any, nbytes: int, *, purpose: str = "block") -> Any:
    """A uint8 tensor of at least ``nbytes`` on ``device``, owned by the
    current stream of that device (any contents)."""
    import torch

    device = torch.device(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    stream = torch.cuda.current_stream(index).cuda_stream
    key = (index, int(stream), purpose)
    with _lock:
        buf = _buffers.get(key)
        if buf is None or buf.numel() < nbytes:
            _buffers.pop(key, None)
            buf = torch.empty(int(nbytes), dtype=torch.uint8, device=torch.device("cuda", index))
            _buffers[key] = buf
        return buf


def release() -> None:
    """Drop every cached workspace (the caching allocator keeps the memory
    until ``torch.cuda.empty_cache()``)."""
    with _lock:
        _buffers.clear()


def manifest() -> dict[str, int]:
    with _lock:
        return {f"cuda:{k[0]}/stream {k[1]:#x}/{k[2]}": int(v.numel()) for k, v in _buffers.items()}
