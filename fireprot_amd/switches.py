"""Per-path disable switches, read once when the package is imported.

The reference lets an operator turn each accelerated path off from the
environment, e.g. ``FIREPROT_DISABLE_CK_ATTENTION`` (ck_attention.py:18-21),
``FIREPROT_DISABLE_LONG_TRIANGLE_ATTENTION`` and
``FIREPROT_DISABLE_LONG_DIRECT_ATTENTION`` (triangle_attention.py:28-33) or
``FIREPROT_DISABLE_RECYCLE_OPS`` (adapters/protenix/hooks.py:33): the
path's capability predicate then rejects every call with a reason and the
caller's native function runs (tests/operators/test_ck_attention.py:44-51).

Here every HIP candidate has its own flag.  A flag is set by the value
``"1"``; the environment is read at import, so a running process keeps the
choice it started with (as the reference's module-level reads do).
``FPX_DISABLE_ALL=1`` turns every path off at once.
"""
from __future__ import annotations

import os

#: flag -> the path it turns off (candidate name or stage hook)
FLAGS: dict[str, str] = {
    "FPX_DISABLE_ATTENTION": "triangle_attention: amd-gfx950-hip-attention-f32",
    "FPX_DISABLE_BLOCK": "triangle_attention_block: amd-gfx950-hip-block-f32",
    "FPX_DISABLE_BLOCK_BF16": "triangle_attention_block: amd-gfx950-hip-block-bf16",
    "FPX_DISABLE_TRIANGLE_MULTIPLICATION":
        "triangle_multiplication: amd-gfx950-hip-triangle-multiplication-f32",
    "FPX_DISABLE_TRANSITION": "transition: amd-gfx950-hip-transition-f32",
    "FPX_DISABLE_OPENFOLD3_ATTENTION": "openfold3 _attention: amd-gfx950-hip-attention-strided-f32",
    "FPX_DISABLE_LAYER_NORM": "pair LayerNorm hook (layer_norm.dispatch_layer_norm)",
    "FPX_DISABLE_QKV_PROJECTION": "q/k/v projection hook (qkv_projection.prepare)",
    "FPX_DISABLE_ATTENTION_GATE": "sigmoid gate hook (attention_gate.wrap_up)",
}

_ALL = os.environ.get("FPX_DISABLE_ALL") == "1"
_STATE: dict[str, bool] = {flag: _ALL or os.environ.get(flag) == "1" for flag in FLAGS}


def disabled(flag: str) -> bool:
    """Whether ``flag`` (a key of ``FLAGS``) was set when the package loaded."""
    return _STATE[flag]


def reason(flag: str) -> str:
    """The rejection reason a predicate reports for a disabled path."""
    return f"disabled by {'FPX_DISABLE_ALL' if _ALL else flag}=1"


def rejection(flag: str) -> tuple[bool, str] | None:
    """``(False, reason)`` when ``flag`` is set, else None."""
    return (False, reason(flag)) if _STATE[flag] else None


def manifest() -> dict[str, bool]:
    return dict(_STATE)
