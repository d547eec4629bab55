"""Shared comparison helpers for the parity tests."""
from __future__ import annotations

import torch

from fireprot_amd import block as hip_block
from oracle import triangle_attention as oracle

# FP32 parity bar: max-abs 1e-4 and rel 1e-4 against the native-order oracle.
F32_ATOL = 1e-4
F32_RTOL = 1e-4


def oracle_params(weights: dict) -> oracle.BlockParams:
    return oracle.BlockParams(**weights)


def hip_weights(weights: dict, device="cuda") -> hip_block.BlockWeights:
    return hip_block.BlockWeights.from_tensors(**weights).to(device)


def report(name: str, actual: torch.Tensor, expected: torch.Tensor) -> dict:
    diff = (actual.double() - expected.double()).abs()
    finite = torch.isfinite(expected)
    stats = {
        "max_abs": diff[finite].max().item() if finite.any() else 0.0,
        "ref_max": expected[finite].abs().max().item() if finite.any() else 0.0,
    }
    print(f"{name}: max|err|={stats['max_abs']:.3e} max|ref|={stats['ref_max']:.3e}", flush=True)
    return stats


def assert_f32_parity(name: str, actual: torch.Tensor, expected: torch.Tensor) -> None:
    actual = actual.detach().cpu()
    expected = expected.detach().cpu()
    report(name, actual, expected)
    torch.testing.assert_close(actual, expected, atol=F32_ATOL, rtol=F32_RTOL, equal_nan=True)


def region_reports(name: str, actual: torch.Tensor, expected: torch.Tensor,
                   valid: int | None, rows: torch.Tensor | None = None) -> None:
    """Report the valid and the padded (masked) outer rows separately."""
    if valid is None:
        report(name, actual, expected)
        return
    index = rows if rows is not None else torch.arange(actual.shape[0])
    keep = index < valid
    if keep.any():
        report(f"{name} [valid rows]", actual[keep], expected[keep])
    if (~keep).any():
        report(f"{name} [padded rows]", actual[~keep], expected[~keep])
