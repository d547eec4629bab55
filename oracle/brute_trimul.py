"""Float64 brute force of triangle multiplication -- TEST INFRASTRUCTURE ONLY.

An independent formulation of the same native arithmetic as
``oracle/triangle_multiplication.py``, as explicit index loops in NumPy
float64 with no torch, no permutes and no batched products:

    zn[i, j, :]  = LayerNorm_in(z[i, j, :])
    ga[i, j, c]  = sigmoid(sum_d zn[i, j, d] w_a_g[c, d] + b_a_g[c])
    a[i, j, c]   = mask[i, j] * ga[i, j, c] * (sum_d zn[i, j, d] w_a_p[c, d] + b_a_p[c])
    b[i, j, c]   = the same with w_b_g, w_b_p
    x[i, j, c]   = sum_k a[i, k, c] b[j, k, c]        (outgoing)
                 = sum_k a[k, i, c] b[k, j, c]        (incoming)
    u[i, j, :]   = sigmoid(w_g zn[i, j] + b_g) * (w_z LayerNorm_out(x[i, j]) + b_z)

(patches/protenix/0001-*.patch:14-46; python/fireprot/backends/amd/
triangle_multiplication.py:136-181, 294-345; kernels/amd/fireprot_amd_ops.cu:
590-602).  It writes the committed fixtures under tests/golden/ and is only
practical for N up to ~12.
"""
from __future__ import annotations

import math

import numpy as np

from .brute import _layer_norm_row


def _sigmoid(x: float) -> float:
    return 1.0 / (1.0 + math.exp(-x))


def _lin(row: np.ndarray, w: np.ndarray, b) -> np.ndarray:
    out = np.empty(w.shape[0], dtype=np.float64)
    for c in range(w.shape[0]):
        acc = 0.0
        for d in range(w.shape[1]):
            acc += float(row[d]) * float(w[c, d])
        out[c] = acc + (float(b[c]) if b is not None else 0.0)
    return out


def update(z: np.ndarray, mask: np.ndarray | None, p: dict, *, outgoing: bool) -> np.ndarray:
    """Return u[N, N, C] in float64 for a tiny pair representation."""
    n = z.shape[0]
    hidden = p["w_a_p"].shape[0]
    zn = np.empty((n, n, z.shape[2]), dtype=np.float64)
    a = np.empty((n, n, hidden), dtype=np.float64)
    b = np.empty((n, n, hidden), dtype=np.float64)
    for i in range(n):
        for j in range(n):
            zn[i, j] = _layer_norm_row(z[i, j], p.get("ln_in_w"), p.get("ln_in_b"),
                                       p.get("eps_in", 1e-5))
            m = 1.0 if mask is None else float(mask[i, j])
            pa = _lin(zn[i, j], p["w_a_p"], p.get("b_a_p"))
            qa = _lin(zn[i, j], p["w_a_g"], p.get("b_a_g"))
            pb = _lin(zn[i, j], p["w_b_p"], p.get("b_b_p"))
            qb = _lin(zn[i, j], p["w_b_g"], p.get("b_b_g"))
            for c in range(hidden):
                a[i, j, c] = m * _sigmoid(qa[c]) * pa[c]
                b[i, j, c] = m * _sigmoid(qb[c]) * pb[c]
    u = np.empty_like(zn)
    for i in range(n):
        for j in range(n):
            x = np.zeros(hidden, dtype=np.float64)
            for c in range(hidden):
                acc = 0.0
                for k in range(n):
                    if outgoing:
                        acc += a[i, k, c] * b[j, k, c]
                    else:
                        acc += a[k, i, c] * b[k, j, c]
                x[c] = acc
            xn = _layer_norm_row(x, p.get("ln_out_w"), p.get("ln_out_b"),
                                 p.get("eps_out", 1e-5))
            out = _lin(xn, p["w_z"], p.get("b_z"))
            gate = _lin(zn[i, j], p["w_g"], p.get("b_g"))
            for c in range(out.shape[0]):
                u[i, j, c] = _sigmoid(gate[c]) * out[c]
    return u
