"""Float64 brute force of the triangle-attention block -- TEST INFRASTRUCTURE ONLY.

An independent formulation of the same native arithmetic as
``oracle/triangle_attention.py``, written as explicit index loops in plain
Python/NumPy float64 with no torch, no permutes and no broadcasting of the
biases.  Each logit is formed element by element from the definitions

    x[a, b, :]      = z[a, b, :]   (starting node)   or  z[b, a, :] (ending node)
    xn[a, b, :]     = LayerNorm(x[a, b, :])                          (0005:32)
    bias[h, a, b]   = sum_c xn[a, b, c] * w_bias[h, c]               (0005:42-45)
    mb[i, k]        = inf * (mask_x[i, k] - 1)                       (0005:36-39)
    q[i, h, j, d]   = sum_c xn[i, j, c] * w_q[h*D + d, c] / sqrt(D)  (0002:34-39)
    logit[i,h,j,k]  = sum_d q[i,h,j,d] * k[i,h,k,d] + mb[i,k] + bias[h, j, k]
    o[i, j, h, d]   = sum_k softmax_k(logit[i, h, j, :])[k] * v[i, h, k, d]
    dz_x[i, j, :]   = w_o @ (o[i, j, :, :].flatten() * sigmoid(w_g @ xn[i, j] + b_g)) + b_o
    dz[a, b]        = dz_x[a, b] (start) or dz_x[b, a] (end)

so an index swap, a transposed operand or a dropped term in the vectorised
oracle shows up as a mismatch.

``logits="f32"`` rounds each logit to float32 at the two native add points,
fl32(fl32(fl32(s) + fl32(mb)) + fl32(bias)) (mask first, then bias:
patches/protenix/0005-*.patch:36-45), and keeps everything else in float64.
That reproduces what the FP32 native path does to fully masked rows: -1e9 has
a float32 spacing of 64, so their logits collapse onto a few values and the
softmax weights follow those ties, which plain float64 does not show.

``rounding="bf16"`` is the native path run on bfloat16 tensors: every
value the native BF16 path stores as a bfloat16 tensor is rounded to bfloat16
(through float32, as torch's bf16 kernels compute in float32 and round once)
at the point the native path stores it -- z, the LayerNorm output, each
linear's output (q, k, v, gate logits, triangle bias, out projection), q
after the 1/sqrt(D) scale, the logits after q k^T, after the mask add and
after the bias add (mask bias bf16(inf * (mask - 1)) itself rounded), the
softmax output, the attention output, sigmoid(g) and the gated product
(kernels/amd/fireprot_pair_softmax.cu:19-26 and
kernels/amd/fireprot_mask_bias.cu:9-22 restate the same points).  The
weights enter rounded to bfloat16; every sum is float64 before its rounding.

It is used to write the committed fixtures under tests/golden/ and is only
practical for N up to ~20.
"""
from __future__ import annotations

import math

import numpy as np


def bf16_round(x):
    """float64 -> float32 -> bfloat16 (round to nearest even), as float64."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    finite = np.isfinite(f)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    out = np.where(finite, rounded.view(np.float32), f).astype(np.float64)
    return out if out.ndim else float(out)


def _layer_norm_row(row: np.ndarray, w, b, eps: float) -> np.ndarray:
    n = len(row)
    mean = 0.0
    for value in row:
        mean += float(value)
    mean /= n
    var = 0.0
    for value in row:
        var += (float(value) - mean) ** 2
    var /= n
    inv = 1.0 / math.sqrt(var + eps)
    out = np.empty(n, dtype=np.float64)
    for c in range(n):
        y = (float(row[c]) - mean) * inv
        if w is not None:
            y *= float(w[c])
        if b is not None:
            y += float(b[c])
        out[c] = y
    return out


def block(z: np.ndarray, mask: np.ndarray | None, params: dict, *, ending: bool,
          logits: str = "f64", rounding: str = "f64") -> np.ndarray:
    """Return dz[N, N, C] in float64 for a tiny pair representation.

    ``params`` holds numpy arrays ``ln_w, ln_b, w_q, w_k, w_v, w_g, b_g,
    w_bias, w_o, b_o`` (torch ``[out, in]`` layout; ``ln_*``, ``b_g``, ``b_o``
    may be None) and floats ``inf``, ``eps``.  ``rounding="bf16"``: the
    native BF16 path (module docstring); ``logits`` is then ignored.
    """
    if logits not in ("f64", "f32"):
        raise ValueError("logits must be 'f64' or 'f32'")
    if rounding not in ("f64", "bf16"):
        raise ValueError("rounding must be 'f64' or 'bf16'")
    bf = rounding == "bf16"
    f32 = logits == "f32" and not bf

    def r(x):  # a value the native path stores: bf16 tensors round it
        return bf16_round(x) if bf else x

    z = r(np.asarray(z, dtype=np.float64))
    n = z.shape[0]
    heads, channels = params["w_bias"].shape
    hd = params["w_q"].shape[0]
    dim = hd // heads
    inf = float(params["inf"])
    eps = float(params["eps"])
    f64 = {k: (None if v is None or isinstance(v, float) else r(np.asarray(v, dtype=np.float64)))
           for k, v in params.items()}

    def x_of(a, b):
        return z[b, a] if ending else z[a, b]

    def mask_x(i, k):
        if mask is None:
            return None
        return float(mask[k, i]) if ending else float(mask[i, k])

    xn = np.empty((n, n, channels))
    for a in range(n):
        for b in range(n):
            xn[a, b] = r(_layer_norm_row(x_of(a, b), f64["ln_w"], f64["ln_b"], eps))

    def project(w, row):
        out = np.zeros(w.shape[0])
        for o in range(w.shape[0]):
            acc = 0.0
            for c in range(w.shape[1]):
                acc += w[o, c] * row[c]
            out[o] = acc
        return out

    bias = np.empty((heads, n, n))
    q = np.empty((n, heads, n, dim))
    k = np.empty((n, heads, n, dim))
    v = np.empty((n, heads, n, dim))
    gate = np.empty((n, n, hd))
    scale = 1.0 / math.sqrt(dim)
    for a in range(n):
        for b in range(n):
            row = xn[a, b]
            pb = r(project(f64["w_bias"], row))
            pq = r(project(f64["w_q"], row))
            pk = r(project(f64["w_k"], row))
            pv = r(project(f64["w_v"], row))
            pg = project(f64["w_g"], row)
            for h in range(heads):
                bias[h, a, b] = pb[h]
                for d in range(dim):
                    # native: q / sqrt(D) on the stored q
                    q[a, h, b, d] = r(pq[h * dim + d] / math.sqrt(dim)) if bf else \
                        pq[h * dim + d] * scale
                    k[a, h, b, d] = pk[h * dim + d]
                    v[a, h, b, d] = pv[h * dim + d]
            for e in range(hd):
                g = r(pg[e] + (0.0 if f64["b_g"] is None else f64["b_g"][e]))
                gate[a, b, e] = r(1.0 / (1.0 + math.exp(-g)))

    dz_x = np.empty((n, n, channels))
    for i in range(n):
        for j in range(n):
            gated = np.empty(hd)
            for h in range(heads):
                row_logits = []
                for kk in range(n):
                    s = 0.0
                    for d in range(dim):
                        s += q[i, h, j, d] * k[i, h, kk, d]
                    m = mask_x(i, kk)
                    if bf:
                        s = r(s)
                        if m is not None:
                            s = r(s + r(inf * r(r(m) - 1.0)))
                        s = r(s + bias[h, j, kk])
                    elif f32:
                        s = float(np.float32(s))
                        if m is not None:
                            mb = float(np.float32(np.float32(inf) * np.float32(m - 1.0)))
                            s = float(np.float32(s + mb))
                        s = float(np.float32(s + float(np.float32(bias[h, j, kk]))))
                    else:
                        if m is not None:
                            s += inf * (m - 1.0)
                        s += bias[h, j, kk]
                    row_logits.append(s)
                top = max(row_logits)
                weights = [math.exp(value - top) for value in row_logits]
                total = sum(weights)
                probs = [r(wk / total) for wk in weights]  # the stored softmax output
                for d in range(dim):
                    acc = 0.0
                    for kk in range(n):
                        acc += probs[kk] * v[i, h, kk, d]
                    gated[h * dim + d] = r(r(acc) * gate[i, j, h * dim + d])
            out = project(f64["w_o"], gated)
            if f64["b_o"] is not None:
                out = out + f64["b_o"]
            dz_x[i, j] = r(out)

    if ending:
        return np.ascontiguousarray(dz_x.transpose(1, 0, 2))
    return dz_x
