"""Write the golden fixtures of the triangle-attention block.

The reference stores no vectors for this path (every reference operator test
compares against a live upstream Protenix call, which is not vendored), so
the fixtures here come from ``oracle/brute.py``: an independent float64
formulation with explicit index loops.  Each fixture holds the inputs (z,
mask, weights; float32) and, for the starting and the ending node, two
expected outputs in float64:

  dz_{start,end}_f64  -- the block in float64 throughout
  dz_{start,end}_f32l -- the same, with every logit rounded to float32 at the
                         native add points (mask, then bias), which is what the
                         FP32 native path does to fully masked rows
  dz_{start,end}_bf16 -- the native path on bfloat16 tensors: every stored
                         intermediate rounded to bfloat16 where the native
                         BF16 path stores it (brute.block rounding="bf16")

Cases (H=4, d=32, c=128):
  n5_plain      N=5, no mask, LN gamma=1/beta=0, no gate/out biases
  n7_tail       N=7, last 2 residues masked, affine LN and gate/out biases
  n9_random_x8  N=9, random {0,1} mask with a fully masked outer row and a
                fully masked key column, triangle-bias weights x8
  n6_order      N=6, W_q and W_k x30 (q.k scores of about +/-46) with
                triangle-bias weights x8 and a fully masked outer row: the
                FP32 rounding of fl(fl(s - 1e9) + bias) differs from
                fl(fl(s + bias) - 1e9) there, so this case pins the native
                mask-then-bias order

Run from the repository root:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from fireprot_amd import workloads  # noqa: E402
from oracle import brute  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def _weights(bias_scale=1.0, affine=False, seed=0):
    w = {k: (None if v is None else v.numpy()) for k, v in
         workloads.make_weights(bias_scale).items()}
    if affine:
        rng = np.random.default_rng(seed)
        w["ln_w"] = (1.0 + 0.1 * rng.standard_normal(128)).astype(np.float32)
        w["ln_b"] = (0.1 * rng.standard_normal(128)).astype(np.float32)
        w["b_g"] = rng.standard_normal(128).astype(np.float32)
        w["b_o"] = (0.1 * rng.standard_normal(128)).astype(np.float32)
    return w


def _case(name, n, mask, weights):
    z = workloads.make_pair(n).numpy()
    params = dict(weights, inf=1e9, eps=1e-5)
    arrays = {"z": z}
    if mask is not None:
        arrays["mask"] = mask.astype(np.float32)
    for key, value in weights.items():
        if value is not None:
            arrays[f"w_{key}" if not key.startswith("w_") else key] = value
    for ending, tag in ((False, "start"), (True, "end")):
        for mode, suffix in (("f64", "f64"), ("f32", "f32l")):
            arrays[f"dz_{tag}_{suffix}"] = brute.block(z, mask, params, ending=ending, logits=mode)
        arrays[f"dz_{tag}_bf16"] = brute.block(z, mask, params, ending=ending, rounding="bf16")
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz", flush=True)


def main():
    _case("n5_plain", 5, None, _weights())
    tail = np.ones((7, 7), dtype=np.float32)
    tail[5:, :] = 0.0
    tail[:, 5:] = 0.0
    _case("n7_tail", 7, tail, _weights(affine=True, seed=7))
    rng = np.random.default_rng(9)
    rand = (rng.random((9, 9)) < 0.7).astype(np.float32)
    rand[4, :] = 0.0      # a fully masked outer row
    rand[:, 6] = 0.0      # a fully masked key column
    rand[0, 0] = 1.0
    _case("n9_random_x8", 9, rand, _weights(bias_scale=8.0))
    big = _weights(bias_scale=8.0)
    big["w_q"] = big["w_q"] * 30.0
    big["w_k"] = big["w_k"] * 30.0
    order = np.ones((6, 6), dtype=np.float32)
    order[2, :] = 0.0
    order[:, 5] = 0.0
    _case("n6_order", 6, order, big)


if __name__ == "__main__":
    main()
