"""Write the golden fixtures of the pair transition.

The reference stores no vectors for this path (its operator tests compare
against the live Protenix module), so the fixtures come from
``oracle/brute_transition.py``: an independent float64 formulation with
explicit loops.  Each fixture holds the inputs (z, weights; float32) and the
float64 output ``out``.

Cases (c = 128, n = 4, weights N(0, 0.05^2) unless stated):
  tr3_plain    z [3, 3, 128], plain LayerNorm
  tr4_affine   z [4, 4, 128], affine LayerNorm, weights N(0, 0.2^2) (SiLU in its
               curved range and saturated tails)

Run from the repository root:  python tests/golden/make_golden_transition.py
"""
from __future__ import annotations

import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from fireprot_amd import workloads  # noqa: E402
from oracle import brute_transition  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent


def _case(name, n, *, std, affine, seed):
    z = workloads.make_pair(n).numpy()
    w = {k: (None if v is None else v.numpy())
         for k, v in workloads.make_transition_weights(std, affine=affine, seed=seed).items()}
    arrays = {"z": z, **{k: v for k, v in w.items() if v is not None}}
    arrays["out"] = brute_transition.transition(z, w)
    np.savez_compressed(OUT / f"{name}.npz", **arrays)
    print(f"wrote {name}.npz", flush=True)


def main():
    _case("tr3_plain", 3, std=0.05, affine=False, seed=31)
    _case("tr4_affine", 4, std=0.2, affine=True, seed=41)


if __name__ == "__main__":
    main()
