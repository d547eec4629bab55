"""CPU oracle for the pair transition -- TEST INFRASTRUCTURE ONLY.

Restates, in plain PyTorch on the CPU, the Pairformer pair transition that
the reference accelerates (Protenix ``Transition`` with n = 4, c_in = 128):

    x   = layernorm1(z)                                  (128 channels)
    a   = linear_no_bias_a(x)                            (128 -> 512)
    b   = linear_no_bias_b(x)                            (128 -> 512)
    out = linear_no_bias(silu(a) * b)                    (512 -> 128)

Reference call sites: python/fireprot/backends/amd/recycle.py:203-227
(``_hip_transition``: LayerNorm, ``transition_projection`` or the two linears
followed by ``silu_mul_f32``, then ``linear_no_bias``), kernels/amd/
fireprot_amd_ops.cu:125-145 (``silu(a) * b`` with ``silu(v) = v / (1 +
exp(-v))``) and :1111-1165 (``project_transition``), the hook at
python/fireprot/adapters/protenix/hooks.py:56-68 (``Transition.forward``),
and recycle.py:360-390 (``dispatch_transition``: the residual stays with the
caller).  Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline``
leg of ``bench.py`` may use this module.

Pinned by the float64 brute force in ``oracle/brute_transition.py``
(committed fixtures under ``tests/golden/``), a closed form (W_b = 0 gives 0),
and planted mistakes (tests/test_oracle_transition.py).
"""
from __future__ import annotations

import dataclasses

import torch

from .triangle_attention import layer_norm, linear

CHANNELS = 128
EXPANSION = 4


@dataclasses.dataclass
class TransitionParams:
    """``layernorm1`` affine (nullable), ``W_a``/``W_b`` ``[512, 128]`` and
    ``W_o`` ``[128, 512]`` in torch ``[out, in]`` layout."""

    ln_w: torch.Tensor | None
    ln_b: torch.Tensor | None
    w_a: torch.Tensor
    w_b: torch.Tensor
    w_o: torch.Tensor
    eps: float = 1e-5


def transition(z: torch.Tensor, p: TransitionParams) -> torch.Tensor:
    """``linear_no_bias(silu(linear_a(LN z)) * linear_b(LN z))``."""
    x = layer_norm(z, p.ln_w, p.ln_b, p.eps)
    a = linear(x, p.w_a)
    b = linear(x, p.w_b)
    return linear(torch.nn.functional.silu(a) * b, p.w_o)


def flops(n_rows: int) -> int:
    """Algorithmic flop over ``n_rows`` pair rows (multiply-add = 2 flop)."""
    hidden = EXPANSION * CHANNELS
    return 2 * n_rows * (2 * CHANNELS * hidden + hidden * CHANNELS)
