"""Float64 brute force of the pair transition -- TEST INFRASTRUCTURE ONLY.

Explicit loops in NumPy float64, independent of ``oracle/transition.py``:

    x[r, :]   = LayerNorm(z[r, :])
    a[r, h]   = sum_c x[r, c] w_a[h, c];   b[r, h] = sum_c x[r, c] w_b[h, c]
    g[r, h]   = a[r, h] / (1 + exp(-a[r, h])) * b[r, h]
    out[r, c] = sum_h g[r, h] w_o[c, h]

(python/fireprot/backends/amd/recycle.py:203-227; kernels/amd/
fireprot_amd_ops.cu:125-145).  It writes the committed fixtures under
tests/golden/ and is meant for a few dozen rows.
"""
from __future__ import annotations

import math

import numpy as np

from .brute import _layer_norm_row


def transition(z: np.ndarray, p: dict) -> np.ndarray:
    rows = z.reshape(-1, z.shape[-1])
    hidden = p["w_a"].shape[0]
    out = np.empty((rows.shape[0], p["w_o"].shape[0]), dtype=np.float64)
    for r in range(rows.shape[0]):
        x = _layer_norm_row(rows[r], p.get("ln_w"), p.get("ln_b"), p.get("eps", 1e-5))
        g = np.empty(hidden, dtype=np.float64)
        for h in range(hidden):
            a = 0.0
            b = 0.0
            for c in range(x.shape[0]):
                a += x[c] * float(p["w_a"][h, c])
                b += x[c] * float(p["w_b"][h, c])
            g[h] = a / (1.0 + math.exp(-a)) * b
        for c in range(out.shape[1]):
            acc = 0.0
            for h in range(hidden):
                acc += g[h] * float(p["w_o"][c, h])
            out[r, c] = acc
    return out.reshape(z.shape[:-1] + (out.shape[1],))
