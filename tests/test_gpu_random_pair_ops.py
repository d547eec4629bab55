"""Seeded sweep of the triangle multiplication and the pair transition,
held to the float64 oracles at the FP32 bar.

Draws (fixed seeds): pair sizes and row counts from 1 to 260, so every
remainder of the kernels' 32-row and 128-row tiles occurs; masks (none,
scattered, a valid prefix, fractional values); LayerNorm affines; biased and
unbiased projections; weight and input scales over two binary orders; both
directions of the multiplication; the in-place residual update (z += update),
which must equal z plus the separate output in float32 bit for bit.  Bar, as
for the attention block
(tests/test_gpu_fp32_accuracy.py): max error against the float64 oracle
within max(2e-6 max|ref|, twice the FP32 oracle's own error).
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import transition as htr
from fireprot_amd import triangle_multiplication as htm
from fireprot_amd import workloads
from oracle import transition as tr
from oracle import triangle_multiplication as tm
from tests.test_gpu_fp32_accuracy import strict_close

pytestmark = pytest.mark.gpu

SIZES = (1, 3, 31, 32, 33, 64, 100, 127, 129, 160, 200, 260)


def _trimul_case(seed: int):
    g = torch.Generator().manual_seed(7000 + seed)
    n = SIZES[seed % len(SIZES)]
    z = torch.randn(n, n, 128, generator=g) * float(torch.empty(1).uniform_(0.25, 4.0, generator=g))
    kind = (seed // 2) % 4
    if kind == 0:
        mask = None
    elif kind == 1:
        mask = (torch.rand(n, n, generator=g) > 0.2).float()
    elif kind == 2:
        valid = int(torch.randint(1, n + 1, (1,), generator=g))
        keep = torch.arange(n) < valid
        mask = (keep[:, None] & keep[None, :]).float()
    else:
        mask = torch.rand(n, n, generator=g)
    std = float(torch.empty(1).uniform_(0.05, 0.2, generator=g))
    w = workloads.make_trimul_weights(std, biases=bool(seed % 3 == 0), affine=True,
                                      seed=500 + seed)
    outgoing = bool(seed % 2)
    accumulate = bool((seed // 3) % 2)
    return n, z, mask, w, outgoing, accumulate


@pytest.mark.parametrize("seed", range(16))
def test_random_trimul_meets_the_fp32_bar(seed):
    n, z, mask, w, outgoing, accumulate = _trimul_case(seed)
    print(f"trimul seed={seed} n={n} outgoing={outgoing} accumulate={accumulate} "
          f"mask={'none' if mask is None else f'{float(mask.mean()):.2f}'}", flush=True)
    weights = htm.TriMulWeights.from_tensors(**w).to("cuda")
    with torch.inference_mode():
        zc = z.cuda()
        m = None if mask is None else mask.cuda()
        update = htm.triangle_multiplication(zc, m, weights, outgoing=outgoing)
        if accumulate:
            # z += update in place: the kernel adds its rounded update to z
            # once, so the result is the float32 sum with the separate update
            want = zc + update
            htm.triangle_multiplication(zc, m, weights, outgoing=outgoing, out=zc, accumulate=True)
            assert torch.equal(zc, want), "in-place update differs from z + update"
        actual = update.cpu()
    p32 = tm.TriMulParams(**w)
    ref32 = tm.update(z, mask, p32, outgoing=outgoing)
    ref64 = tm.update(z.double(), None if mask is None else mask.double(), p32.to(torch.float64),
                      outgoing=outgoing)
    strict_close(f"trimul seed {seed} n={n}", actual, ref64, ref32)


def _transition_case(seed: int):
    g = torch.Generator().manual_seed(8000 + seed)
    rows = SIZES[seed % len(SIZES)]
    cols = SIZES[(seed * 5 + 3) % len(SIZES)]
    z = torch.randn(rows, cols, 128, generator=g) * float(torch.empty(1).uniform_(0.25, 4.0,
                                                                                     generator=g))
    std = float(torch.empty(1).uniform_(0.02, 0.1, generator=g))
    w = workloads.make_transition_weights(std, affine=bool(seed % 2 == 0), seed=600 + seed)
    accumulate = bool((seed // 2) % 2)
    return z, w, accumulate


@pytest.mark.parametrize("seed", range(12))
def test_random_transition_meets_the_fp32_bar(seed):
    z, w, accumulate = _transition_case(seed)
    print(f"transition seed={seed} shape={tuple(z.shape[:2])} accumulate={accumulate}", flush=True)
    weights = htr.TransitionWeights.from_tensors(**w).to("cuda")
    with torch.inference_mode():
        zc = z.cuda()
        update = htr.transition(zc, weights)
        if accumulate:
            want = zc + update
            htr.transition(zc, weights, out=zc, accumulate=True)
            assert torch.equal(zc, want), "in-place update differs from z + update"
        actual = update.cpu()
    ref32 = tr.transition(z, tr.TransitionParams(**w))
    w64 = {k: (v.double() if torch.is_tensor(v) else v) for k, v in w.items()}
    ref64 = tr.transition(z.double(), tr.TransitionParams(**w64))
    strict_close(f"transition seed {seed} {tuple(z.shape[:2])}", actual, ref64, ref32)
