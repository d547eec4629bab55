"""CPU oracle for triangle multiplication -- TEST INFRASTRUCTURE ONLY.

Restates, in plain PyTorch on the CPU, the native arithmetic of the Pairformer
triangle multiplicative update (outgoing and incoming) that the reference
accelerates.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and never as the code that is
measured or shipped.

Reference call sites (paths relative to the reference checkout):

* module call and in-place contract -- patches/protenix/0001-*.patch:14-46
  (``TriangleMultiplicativeUpdate.forward(z, mask, inplace_safe,
  _add_with_inplace)``), python/fireprot/backends/amd/
  triangle_multiplication.py:73-92 (``z.add_(update)`` when adding,
  ``z.copy_(update)`` otherwise; the result aliases z)
* op order of the update -- triangle_multiplication.py:136-181:
  ``normalized = layer_norm_in(z)``;
  ``a = mask * sigmoid(linear_a_g(normalized)) * linear_a_p(normalized)``
  (the mask multiplies first, as in the native ``a = mask; a = a * sigmoid(..);
  a = a * ..``); ``b`` likewise; ``x = combine(a, b)``;
  ``x = linear_z(layer_norm_out(x))``; ``x = sigmoid(linear_g(normalized)) * x``
* the contraction -- docs/protenix-packed-triangle.md (flow, step 4) and
  triangle_multiplication.py:318 (``packed_bmm(a, b, module._outgoing)``):
  outgoing ``x[i, j, c] = sum_k a[i, k, c] b[j, k, c]`` (``a @ b^T`` per
  channel), incoming ``x[i, j, c] = sum_k a[k, i, c] b[k, j, c]``
  (``a^T @ b``)
* residual value -- kernels/amd/fireprot_amd_ops.cu:590-602
  (``add ? z + sigmoid(g) * x : sigmoid(g) * x``)
* LayerNorm -- torch.nn.LayerNorm over the last axis (eps 1e-5), as the
  reference tests select with LAYERNORM_TYPE=torch
  (tests/operators/test_triangle_multiplication.py:8)

The upstream Protenix module is not vendored in the reference and is not
installed here.  This restatement is pinned by the float64 brute force in
``oracle/brute_trimul.py`` (explicit index loops; committed fixtures under
``tests/golden/``), by closed forms (a zero mask gives the constant
``sigmoid(g) * (ln_out_b W_z^T + b_z)``) and by the direction identity
``incoming(z; a, b) = T(outgoing(T(z); b, a))`` with the gate read in the
same frame (tests/test_oracle_trimul.py).
"""
from __future__ import annotations

import dataclasses

import torch

from .triangle_attention import layer_norm, linear

CHANNELS = 128
HIDDEN = 128


@dataclasses.dataclass
class TriMulParams:
    """Weights of one triangle multiplicative update, torch ``[out, in]``.

    Protenix builds every projection without a bias term; the optional biases
    cover OpenFold-style modules that carry them.
    """

    ln_in_w: torch.Tensor | None
    ln_in_b: torch.Tensor | None
    w_a_p: torch.Tensor
    w_a_g: torch.Tensor
    w_b_p: torch.Tensor
    w_b_g: torch.Tensor
    ln_out_w: torch.Tensor | None
    ln_out_b: torch.Tensor | None
    w_z: torch.Tensor
    w_g: torch.Tensor
    b_a_p: torch.Tensor | None = None
    b_a_g: torch.Tensor | None = None
    b_b_p: torch.Tensor | None = None
    b_b_g: torch.Tensor | None = None
    b_z: torch.Tensor | None = None
    b_g: torch.Tensor | None = None
    eps_in: float = 1e-5
    eps_out: float = 1e-5

    def to(self, dtype: torch.dtype) -> "TriMulParams":
        fields = {f.name: getattr(self, f.name) for f in dataclasses.fields(self)}
        return TriMulParams(**{k: (v.to(dtype) if isinstance(v, torch.Tensor) else v)
                               for k, v in fields.items()})


def gated_projections(z: torch.Tensor, mask: torch.Tensor | None,
                      p: TriMulParams) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """``normalized``, ``a`` and ``b`` ``[N, N, 128]`` (triangle_multiplication.py:155-170)."""
    normalized = layer_norm(z, p.ln_in_w, p.ln_in_b, p.eps_in)
    m = (torch.ones(z.shape[:-1], dtype=z.dtype) if mask is None else mask.to(z.dtype))
    m = m.unsqueeze(-1)
    a = m * torch.sigmoid(linear(normalized, p.w_a_g, p.b_a_g))
    a = a * linear(normalized, p.w_a_p, p.b_a_p)
    b = m * torch.sigmoid(linear(normalized, p.w_b_g, p.b_b_g))
    b = b * linear(normalized, p.w_b_p, p.b_b_p)
    return normalized, a, b


def combine(a: torch.Tensor, b: torch.Tensor, *, outgoing: bool) -> torch.Tensor:
    """The per-channel contraction, returned as ``[N, N, 128]``.

    outgoing: ``x[i, j] = sum_k a[i, k] b[j, k]``; incoming:
    ``x[i, j] = sum_k a[k, i] b[k, j]`` (one matmul per channel).
    """
    ac = a.permute(2, 0, 1)  # [c, d0, d1]
    bc = b.permute(2, 0, 1)
    if outgoing:
        x = torch.matmul(ac, bc.transpose(1, 2))
    else:
        x = torch.matmul(ac.transpose(1, 2), bc)
    return x.permute(1, 2, 0)


def update(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulParams, *,
           outgoing: bool, rows: torch.Tensor | None = None) -> torch.Tensor:
    """The module's update ``sigmoid(linear_g(LN_in z)) * linear_z(LN_out(x))``.

    ``rows`` restricts the output to those first-index rows ``i`` (each output
    row needs all of ``b`` and one row, or column, of ``a``); the result is then
    ``[len(rows), N, 128]`` and equals ``update(...)[rows]``, which
    tests/test_oracle_trimul.py checks.
    """
    normalized, a, b = gated_projections(z, mask, p)
    if rows is None:
        x = combine(a, b, outgoing=outgoing)
    else:
        a_rows = a[rows] if outgoing else a[:, rows].transpose(0, 1)  # [R, k, c]
        b_k = b if outgoing else b.transpose(0, 1)                      # [j, k, c]
        x = torch.matmul(a_rows.permute(2, 0, 1), b_k.permute(2, 1, 0)).permute(1, 2, 0)
        normalized = normalized[rows]
    del a, b
    x = linear(layer_norm(x, p.ln_out_w, p.ln_out_b, p.eps_out), p.w_z, p.b_z)
    return torch.sigmoid(linear(normalized, p.w_g, p.b_g)) * x


def forward(z: torch.Tensor, mask: torch.Tensor | None, p: TriMulParams, *, outgoing: bool,
            add: bool) -> torch.Tensor:
    """In-place module contract: returns ``z + update`` (add) or ``update``."""
    u = update(z, mask, p, outgoing=outgoing)
    return z + u if add else u


def flops(n: int) -> dict[str, int]:
    """Algorithmic flop of one update (multiply-add = 2 flop)."""
    proj = 2 * n * n * CHANNELS * HIDDEN * 4       # a_p, a_g, b_p, b_g
    contract = 2 * n ** 3 * HIDDEN                 # one N x N x N product per channel
    out = 2 * n * n * (HIDDEN * CHANNELS + CHANNELS * CHANNELS)  # linear_z, linear_g
    return {"projections": proj, "contraction": contract, "output": out,
            "total": proj + contract + out}
