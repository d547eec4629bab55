"""Write the golden fixtures of triangle multiplication.

The reference stores no vectors for this path (its operator tests compare
against a live upstream Protenix module, which is not vendored), so the
fixtures come from ``oracle/brute_trimul.py``: an independent float64
formulation with explicit index loops.  Each fixture holds the inputs (z,
mask, weights; float32) and the float64 update of both directions:

  u_out -- outgoing  x[i, j] = sum_k a[i, k] b[j, k]
  u_in  -- incoming  x[i, j] = sum_k a[k, i] b[k, j]

Cases (c_z = c_hidden = 128, weights N(0, 0.1^2)):
  t5_plain        N=5, no mask, plain LayerNorms, no projection biases
  t6_mask_affine  N=6, random {0,1} mask with a fully masked row and column,
                  affine LayerNorms and biases on all six projections
  t7_tail         N=7, last 2 residues masked on both axes, no biases

Run from the repository root:  python tests/golden/make_golden_trimul.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from fireprot_amd import workloads  # noqa: E402
from oracle import brute_trimul  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def _case(name, n, mask, *, biases, affine, seed):
    z = workloads.make_pair(n).numpy()
    w = {k: (None if v is None else v.numpy())
         for k, v in workloads.make_trimul_weights(biases=biases, affine=affine,
                                                   seed=seed).items()}
    arrays = {"z": z}
    if mask is not None:
        arrays["mask"] = mask.astype(np.float32)
    arrays.update({k: v for k, v in w.items() if v is not None})
    arrays["u_out"] = brute_trimul.update(z, mask, w, outgoing=True)
    arrays["u_in"] = brute_trimul.update(z, mask, w, outgoing=False)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz", flush=True)


def main():
    _case("t5_plain", 5, None, biases=False, affine=False, seed=51)
    rng = np.random.default_rng(6)
    rand = (rng.random((6, 6)) < 0.7).astype(np.float32)
    rand[2, :] = 0.0
    rand[:, 4] = 0.0
    _case("t6_mask_affine", 6, rand, biases=True, affine=True, seed=61)
    tail = np.ones((7, 7), dtype=np.float32)
    tail[5:, :] = 0.0
    tail[:, 5:] = 0.0
    _case("t7_tail", 7, tail, biases=False, affine=False, seed=71)


if __name__ == "__main__":
    main()
