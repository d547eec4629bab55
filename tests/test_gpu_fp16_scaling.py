"""Power-of-two scaled fp16 planes keep FP32 accuracy across magnitudes.

The projections and GEMMs of the triangle multiplication and the pair
transition hold their operands as fp16 (hi, lo) planes scaled by powers of
two: LayerNorm rows by one exponent from the LN affine, weight rows per
output channel, the contraction's a and b rows per (channel, row) from the
row maxima the projection records, and the transition's hidden layer by the
launch's max.  Scaling the weights by factors far from 1 moves every
exponent; the results must then still match the float64 oracle to FP32
level: within 2e-6 of the largest output (the bar of the brute-force
fixtures) or, where the case is ill-conditioned, within twice the error of
the same oracle evaluated in float32.  A NaN in z must reach exactly the
outputs it reaches in the oracle.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import workloads
from fireprot_amd import transition as htr
from fireprot_amd import triangle_multiplication as htm
from oracle import transition as tr
from oracle import triangle_multiplication as tm

pytestmark = pytest.mark.gpu


def _tr64(w):
    return tr.TransitionParams(**{k: v.double() if torch.is_tensor(v) else v for k, v in w.items()})


def _close(name, actual, expected, fp32=None, tol=2e-6):
    """expected: float64 oracle; fp32: the oracle in float32 (optional)."""
    expected = expected.double()
    err = (actual.double() - expected).abs().max().item()
    ref = expected.abs().max().item()
    bar = tol * ref
    if fp32 is not None:
        bar = max(bar, 2.0 * (fp32.double() - expected).abs().max().item())
    print(f"{name}: max|err|={err:.3e} max|ref|={ref:.3e} bar={bar:.3e}", flush=True)
    assert err <= bar


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("std", [1e-3, 0.1, 30.0])
def test_trimul_weight_scales(std, outgoing):
    n = 80
    z = workloads.make_pair(n)
    g = torch.Generator().manual_seed(7)
    mask = (torch.rand(n, n, generator=g) < 0.8).float()
    w = workloads.make_trimul_weights(std=std, biases=True, affine=True)
    with torch.inference_mode():
        actual = htm.triangle_multiplication(z.cuda(), mask.cuda(),
                                             htm.TriMulWeights.from_tensors(**w).to("cuda"),
                                             outgoing=outgoing).cpu()
    expected = tm.update(z.double(), mask.double(), tm.TriMulParams(**w).to(torch.float64),
                         outgoing=outgoing)
    fp32 = tm.update(z, mask, tm.TriMulParams(**w), outgoing=outgoing)
    _close(f"trimul std={std} outgoing={outgoing}", actual, expected, fp32)


def test_trimul_nan_reaches_the_oracle_pattern():
    n = 48
    z = workloads.make_pair(n)
    z[5, 9, 3] = float("nan")
    w = workloads.make_trimul_weights()
    with torch.inference_mode():
        actual = htm.triangle_multiplication(z.cuda(), None,
                                             htm.TriMulWeights.from_tensors(**w).to("cuda"),
                                             outgoing=True).cpu()
    expected = tm.update(z.double(), None, tm.TriMulParams(**w).to(torch.float64), outgoing=True)
    assert torch.isnan(expected).any()
    assert torch.equal(torch.isnan(actual), torch.isnan(expected))
    finite = ~torch.isnan(expected)
    _close("trimul nan (finite part)", actual[finite], expected[finite])


@pytest.mark.parametrize("std", [1e-3, 0.05, 20.0])
def test_transition_weight_scales(std):
    g = torch.Generator().manual_seed(11)
    z = torch.randn(37, 41, 128, generator=g)
    w = workloads.make_transition_weights(std=std, affine=True)
    with torch.inference_mode():
        actual = htr.transition(z.cuda(), htr.TransitionWeights.from_tensors(**w).to("cuda")).cpu()
    expected = tr.transition(z.double(), _tr64(w))
    _close(f"transition std={std}", actual, expected, tr.transition(z, tr.TransitionParams(**w)))


def test_transition_output_weight_rows_of_different_magnitudes():
    """W_o rows scaled from 1e-4 to 1e4: each output channel keeps its own
    exponent."""
    g = torch.Generator().manual_seed(12)
    z = torch.randn(20, 33, 128, generator=g)
    w = workloads.make_transition_weights(affine=True)
    w["w_o"] = w["w_o"] * torch.logspace(-4, 4, 128)[:, None]
    with torch.inference_mode():
        actual = htr.transition(z.cuda(), htr.TransitionWeights.from_tensors(**w).to("cuda")).cpu()
    expected = tr.transition(z.double(), _tr64(w))
    fp32 = tr.transition(z, tr.TransitionParams(**w))
    for c in (0, 64, 127):
        _close(f"transition channel {c}", actual[..., c], expected[..., c], fp32[..., c])
