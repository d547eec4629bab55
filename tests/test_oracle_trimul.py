"""Pins of the triangle-multiplication oracle (CPU).

``oracle/triangle_multiplication.py`` is checked against the float64
brute-force fixtures (explicit index loops, tests/golden/t*.npz), a closed
form, the outgoing/incoming direction identity, relabelling equivariance, and
planted mistakes that each check must reject.
"""
from __future__ import annotations

import pathlib

import numpy as np
import pytest
import torch

from fireprot_amd import workloads
from oracle import brute_trimul
from oracle import triangle_multiplication as tm

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
CASES = ("t5_plain", "t6_mask_affine", "t7_tail")
FIELDS = ("ln_in_w", "ln_in_b", "w_a_p", "w_a_g", "w_b_p", "w_b_g", "ln_out_w", "ln_out_b",
          "w_z", "w_g", "b_a_p", "b_a_g", "b_b_p", "b_b_g", "b_z", "b_g")


def load_trimul_case(name: str, dtype=torch.float64):
    with np.load(GOLDEN / f"{name}.npz") as data:
        arrays = {k: torch.from_numpy(data[k]) for k in data.files}
    z = arrays["z"].to(dtype)
    mask = arrays["mask"].to(dtype) if "mask" in arrays else None
    params = tm.TriMulParams(**{k: (arrays[k].to(dtype) if k in arrays else None)
                                for k in FIELDS})
    return z, mask, params, arrays["u_out"], arrays["u_in"]


def params_of(weights: dict, dtype=torch.float32) -> tm.TriMulParams:
    return tm.TriMulParams(**{k: (None if v is None else v.to(dtype))
                              for k, v in weights.items()})


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_brute_force_fixtures(name):
    z, mask, params, u_out, u_in = load_trimul_case(name)
    torch.testing.assert_close(tm.update(z, mask, params, outgoing=True), u_out,
                               atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(tm.update(z, mask, params, outgoing=False), u_in,
                               atol=1e-10, rtol=1e-10)
    # the FP32 oracle (the parity reference of the GPU tests) to FP32 accuracy
    z32, m32, p32, _, _ = load_trimul_case(name, torch.float32)
    torch.testing.assert_close(tm.update(z32, m32, p32, outgoing=True).double(), u_out,
                               atol=2e-6, rtol=1e-5)


def test_fixtures_differ_between_directions_and_cases():
    _, _, _, u_out, u_in = load_trimul_case("t6_mask_affine")
    assert (u_out - u_in).abs().max() > 1e-2


def test_zero_mask_closed_form():
    """mask = 0: a = b = 0, x = 0, LN_out(0) = ln_out_b, so the update is
    sigmoid(W_g LN_in(z) + b_g) * (W_z ln_out_b + b_z) at every pair."""
    n = 5
    z = workloads.make_pair(n).double()
    p = params_of(workloads.make_trimul_weights(biases=True, affine=True), torch.float64)
    mask = torch.zeros(n, n, dtype=torch.float64)
    zn = torch.nn.functional.layer_norm(z, (128,), p.ln_in_w, p.ln_in_b, 1e-5)
    expected = torch.sigmoid(zn @ p.w_g.T + p.b_g) * (p.w_z @ p.ln_out_b + p.b_z)
    for outgoing in (True, False):
        torch.testing.assert_close(tm.update(z, mask, p, outgoing=outgoing), expected,
                                   atol=1e-12, rtol=1e-12)
    brute = brute_trimul.update(z.numpy(), mask.numpy(),
                                {k: (None if getattr(p, k) is None else getattr(p, k).numpy())
                                 for k in FIELDS}, outgoing=True)
    torch.testing.assert_close(torch.from_numpy(brute), expected, atol=1e-12, rtol=1e-12)


def _swap_ab(p: tm.TriMulParams) -> tm.TriMulParams:
    return tm.TriMulParams(**{**p.__dict__, "w_a_p": p.w_b_p, "w_a_g": p.w_b_g,
                              "w_b_p": p.w_a_p, "w_b_g": p.w_a_g, "b_a_p": p.b_b_p,
                              "b_a_g": p.b_b_g, "b_b_p": p.b_a_p, "b_b_g": p.b_a_g})


def test_incoming_is_transposed_outgoing_with_swapped_branches():
    n = 9
    z = workloads.make_pair(n).double()
    mask = (torch.rand(n, n, generator=torch.Generator().manual_seed(3)) < 0.8).double()
    p = params_of(workloads.make_trimul_weights(biases=True), torch.float64)
    incoming = tm.update(z, mask, p, outgoing=False)
    mirrored = tm.update(z.transpose(0, 1).contiguous(), mask.t().contiguous(), _swap_ab(p),
                         outgoing=True).transpose(0, 1)
    torch.testing.assert_close(incoming, mirrored, atol=1e-12, rtol=1e-12)


def test_relabelling_equivariance():
    n = 8
    z = workloads.make_pair(n).double()
    mask = (torch.rand(n, n, generator=torch.Generator().manual_seed(4)) < 0.8).double()
    p = params_of(workloads.make_trimul_weights(), torch.float64)
    perm = torch.randperm(n, generator=torch.Generator().manual_seed(5))
    for outgoing in (True, False):
        base = tm.update(z, mask, p, outgoing=outgoing)
        moved = tm.update(z[perm][:, perm], mask[perm][:, perm], p, outgoing=outgoing)
        torch.testing.assert_close(moved, base[perm][:, perm], atol=1e-12, rtol=1e-12)


def test_row_subset_matches_full_update():
    n = 10
    z = workloads.make_pair(n).double()
    mask = (torch.rand(n, n, generator=torch.Generator().manual_seed(8)) < 0.8).double()
    p = params_of(workloads.make_trimul_weights(biases=True), torch.float64)
    rows = torch.tensor([0, 3, 9, 4])
    for outgoing in (True, False):
        full = tm.update(z, mask, p, outgoing=outgoing)
        part = tm.update(z, mask, p, outgoing=outgoing, rows=rows)
        torch.testing.assert_close(part, full[rows], atol=1e-12, rtol=1e-12)


def test_forward_adds_or_overwrites():
    z, mask, params, u_out, _ = load_trimul_case("t7_tail")
    torch.testing.assert_close(tm.forward(z, mask, params, outgoing=True, add=True), z + u_out,
                               atol=1e-10, rtol=1e-10)
    torch.testing.assert_close(tm.forward(z, mask, params, outgoing=True, add=False), u_out,
                               atol=1e-10, rtol=1e-10)


def _planted_combine(kind):
    def combine(a, b, *, outgoing):
        ac, bc = a.permute(2, 0, 1), b.permute(2, 0, 1)
        if kind == "transposed_b":       # sum_k a[i, k] b[k, j]
            x = torch.matmul(ac, bc)
        elif kind == "swapped_dirs":     # incoming formula for outgoing
            x = torch.matmul(ac.transpose(1, 2), bc)
        return x.permute(1, 2, 0)
    return combine


@pytest.mark.parametrize("kind", ["transposed_b", "swapped_dirs"])
def test_planted_contraction_mistakes_are_rejected(kind, monkeypatch):
    z, mask, params, u_out, _ = load_trimul_case("t6_mask_affine")
    monkeypatch.setattr(tm, "combine", _planted_combine(kind))
    wrong = tm.update(z, mask, params, outgoing=True)
    assert (wrong - u_out).abs().max() > 1e-3


def test_planted_gate_mistakes_are_rejected():
    z, mask, params, u_out, _ = load_trimul_case("t6_mask_affine")
    normalized, a, b = tm.gated_projections(z, mask, params)
    x = tm.combine(a, b, outgoing=True)
    xo = tm.linear(tm.layer_norm(x, params.ln_out_w, params.ln_out_b, 1e-5), params.w_z,
                   params.b_z)
    gate_raw_z = torch.sigmoid(tm.linear(z, params.w_g, params.b_g)) * xo     # un-normalised z
    no_mask = tm.update(z, None, params, outgoing=True)                       # mask dropped
    for wrong in (gate_raw_z, no_mask):
        assert (wrong - u_out).abs().max() > 1e-3
