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


@pytest.mark.parametrize("seed", range(16))
def test_random_core_masked_meets_the_fp32_bar(seed):
    """The FP32-matrix-core entry behind the reference-ABI names,
    fpx_attn_core_masked, on the same kind of draws: N a multiple of 4 from 4
    to 260, padded bias rows, binary, moderate or no mask biases."""
    from fireprot_amd import _native

    g = torch.Generator().manual_seed(6500 + seed)
    n = 4 * int(torch.randint(1, 66, (1,), generator=g))
    batch = int(torch.randint(1, 17, (1,), generator=g))
    mask = ("binary", "moderate", "none")[seed % 3]
    q, k, v, mb, bias = make_case(batch, n, 6600 + seed, mask=mask)
    bias = bias * float(torch.empty(1).uniform_(0.25, 4.0, generator=g))
    pad = 4 * int(torch.randint(0, 5, (1,), generator=g))
    print(f"core seed={seed} batch={batch} n={n} mask={mask} bias row stride {n + pad}",
          flush=True)

    def head_last(t):  # [B, 4, N, 32] values in [B, N, 4, 32] memory
        return t.transpose(1, 2).contiguous().cuda()

    qc, kc, vc = (head_last(t) for t in (q, k, v))
    bias_rows = torch.zeros(4, n, n + pad)
    bias_rows[:, :, :n] = bias[0]
    bc = bias_rows.cuda()
    mc = mb[:, 0, 0, :].contiguous().cuda() if mask != "none" else None
    out = torch.full((batch, n, 4, 32), float("nan"), device="cuda")
    code = _native.library().fpx_attn_core_masked(
        qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), None if mc is None else mc.data_ptr(),
        n if mc is not None else 0, bc.data_ptr(), n + pad, out.data_ptr(), batch, n,
        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert code == 0
    actual = out.cpu().transpose(1, 2)  # [B, 4, N, 32]
    biases32 = [bias] if mask == "none" else [mb, bias]
    dead = (mb[:, 0, 0, :] <= -1e8).all(dim=-1) if mask != "none" else torch.zeros(batch, dtype=torch.bool)
    for region, sel in (("open", ~dead), ("masked", dead)):
        if not sel.any():
            continue
        b = torch.nonzero(sel).flatten()
        bl = [t[b] if t.shape[0] == batch and t is not bias else t for t in biases32]
        ref32 = oracle.attention_core(q[b], k[b], v[b], bl)
        ref64 = oracle.attention_core(q[b].double(), k[b].double(), v[b].double(),
                                      [t.double() for t in bl], logits_f32=(region == "masked"))
        strict_close(f"core seed {seed} {region}", actual[b], ref64, ref32)
