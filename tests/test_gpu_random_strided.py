"""Seeded sweep of the strided attention (fpx_attn_strided: the OpenFold3
consumer and the registered operator route), held to the float64 oracle at
the FP32 bar.

Draws (fixed seeds): batch 1-24 and N 1-260, so every remainder of the 32-key
tiles and 128-query work-groups occurs; binary masks with fully masked rows,
moderate additive mask values, or none; every triangle-bias layout OpenFold3
hands over (head-first or head-last, as is or transposed), per-row or
transposed mask views, head-last or contiguous q/k/v; q, k and bias scales
over two binary orders.  Bar, as for the block (tests/test_gpu_fp32_accuracy.py):
max error against float64 within max(2e-6 max|ref|, twice the FP32 oracle's
own error); rows whose keys are all masked against float64 with the logits
rounded to float32 where the native path adds them (their -1e9 ties).
"""
from __future__ import annotations

import pytest
import torch

from oracle import triangle_attention as oracle
from tests.test_gpu_fp32_accuracy import strict_close
from tests.test_gpu_openfold3 import BIAS_LAYOUTS, make_case, run

pytestmark = pytest.mark.gpu

SIZES = (1, 2, 31, 33, 64, 97, 128, 129, 200, 257, 260)


def _case(seed: int):
    g = torch.Generator().manual_seed(6000 + seed)
    n = SIZES[seed % len(SIZES)]
    batch = int(torch.randint(1, 25, (1,), generator=g))
    mask = ("binary", "moderate", "none")[seed % 3]
    q, k, v, mb, bias = make_case(batch, n, 6100 + seed, mask=mask)
    q = q * float(torch.empty(1).uniform_(0.5, 2.0, generator=g))
    k = k * float(torch.empty(1).uniform_(0.5, 2.0, generator=g))
    bias = bias * float(torch.empty(1).uniform_(0.25, 4.0, generator=g))
    layouts = dict(bias_layout=BIAS_LAYOUTS[seed % 4],
                   mask_layout=("rows", "transposed")[(seed // 4) % 2],
                   qkv=("head_last", "contiguous")[(seed // 2) % 2])
    return batch, n, mask, (q, k, v, mb, bias), layouts


@pytest.mark.parametrize("seed", range(24))
def test_random_strided_meets_the_fp32_bar(seed):
    batch, n, mask, (q, k, v, mb, bias), layouts = _case(seed)
    print(f"strided seed={seed} batch={batch} n={n} mask={mask} {layouts}", flush=True)
    actual = run(q, k, v, mb, bias, **layouts)
    dead = (mb[:, 0, 0, :] <= -1e8).all(dim=-1)  # [B]: rows whose keys are all masked
    for region, sel in (("open", ~dead), ("masked", dead)):
        if not sel.any():
            continue
        b = torch.nonzero(sel).flatten()
        ref32 = oracle.attention_core(q[b], k[b], v[b], [mb[b], bias])
        ref64 = oracle.attention_core(q[b].double(), k[b].double(), v[b].double(),
                                      [mb[b].double(), bias.double()],
                                      logits_f32=(region == "masked"))
        strict_close(f"strided seed {seed} {region}", actual[b], ref64, ref32)
