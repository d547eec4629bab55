"""Trailing fully masked key tiles are left out of the attention on rows that
have an unmasked key, when the prepare stage's magnitude record bounds the
logits.  Their weights are exactly 0, so the result must be bit-identical to
visiting them.

A mask bias of -1e9 (the block's default inf) puts the masked tiles at or
below -2^29 and lets them be skipped; -1e8 keeps them visited while their
weights are still exactly 0.  Outer rows that have an unmasked key must
therefore agree bit for bit between the two, and both with the oracle.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import block as hip_block
from fireprot_amd import workloads
from oracle import triangle_attention as oracle
from tests.helpers import assert_f32_parity, oracle_params

pytestmark = pytest.mark.gpu


def _run(z, mask, w, ending, inf):
    weights = hip_block.BlockWeights.from_tensors(**w, inf=inf).to("cuda")
    with torch.inference_mode():
        out = hip_block.triangle_attention_block(z.cuda(), mask.cuda(), weights, ending=ending)
        torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("n,valid", [(300, 200), (1000, 880)])
def test_skipped_tail_tiles_are_bit_identical(n, valid, ending):
    print(f"case n={n} valid={valid} ending={ending}", flush=True)
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights()
    skipped = _run(z, mask, w, ending, 1e9)
    visited = _run(z, mask, w, ending, 1e8)
    # outer rows with an unmasked key: i < valid in the block's own frame
    rows_s = skipped.transpose(0, 1) if ending else skipped
    rows_v = visited.transpose(0, 1) if ending else visited
    assert torch.equal(rows_s[:valid], rows_v[:valid])
    if n <= 300:
        expected = oracle.block(z, mask, oracle_params(w), ending=ending)
        assert_f32_parity(f"skip n={n} ending={ending}", skipped, expected)
    else:
        rows = torch.tensor([0, 1, valid // 2, valid - 1, valid, n - 1])
        expected = oracle.block(z, mask, oracle_params(w), ending=ending, outer_rows=rows)
        # the oracle returns the selected outer rows in the block's own frame
        assert_f32_parity(f"skip n={n} ending={ending} rows", rows_s[rows], expected)


def test_non_finite_masked_key_still_poisons_its_rows():
    """A NaN at a masked pair makes k, v and the triangle bias of that pair
    NaN; the native path then returns NaN wherever that key or bias enters a
    softmax.  The magnitude record sees the NaN and keeps every tile visited."""
    n, valid = 160, 100
    z = workloads.make_pair(n)
    z[3, 130, 7] = float("nan")  # row 3 (unmasked), key 130 (masked tail)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights()
    expected = oracle.block(z, mask, oracle_params(w), ending=False)
    assert torch.isnan(expected).any()
    actual = _run(z, mask, w, False, 1e9)
    assert torch.equal(torch.isnan(actual), torch.isnan(expected))
    assert_f32_parity("nan at masked key", actual, expected)
