"""Seeded sweep of pair sizes, masks and weights, held to the float64 oracle.

The fixtures and the C2-C5 cases cover chosen shapes; this sweep draws the
rest at random (fixed seeds): pair sizes from 1 to 260, so every remainder
of the 32-key tiles and 128-query work-groups occurs, per-row valid lengths,
scattered masked keys, fully masked rows, a fractional mask value, random
LayerNorm affines and weight scales, and both nodes.  Every output row meets
the FP32 bar of tests/test_gpu_fp32_accuracy.py against the float64 oracle:
rows with an unmasked key against plain float64, fully masked rows (their
-1e9 ties) and the draws with a fractional mask value (a -5e8 mask bias,
whose FP32 spacing of 32 swallows the products) against float64 with the
logits rounded to float32 where the native path adds them.  The BF16
storage path is held to the FP32 oracle on the same bf16-rounded inputs:
within the BF16 bar of tests/test_gpu_bf16.py, or within twice the error of
the native BF16 path (``oracle.block_bf16``) where that is larger.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import block as hip_block
from fireprot_amd import workloads
from oracle import triangle_attention as oracle
from tests.helpers import hip_weights, oracle_params
from tests.test_gpu_fp32_accuracy import strict_close

pytestmark = pytest.mark.gpu

SIZES = (1, 2, 5, 31, 32, 33, 64, 97, 127, 128, 129, 160, 191, 224, 257, 260)


def _case(seed: int):
    g = torch.Generator().manual_seed(9000 + seed)
    n = SIZES[seed % len(SIZES)]
    z = torch.randn(n, n, 128, generator=g) * float(torch.empty(1).uniform_(0.3, 3.0, generator=g))
    kind = (seed + seed // len(SIZES)) % 4
    mask = torch.ones(n, n)
    if kind == 0:  # a valid prefix per row and per column (padded residues)
        valid = int(torch.randint(1, n + 1, (1,), generator=g))
        keep = torch.arange(n) < valid
        mask = (keep[:, None] & keep[None, :]).float()
    elif kind == 1:  # ragged per-row lengths, some rows fully masked
        lengths = torch.randint(0, n + 1, (n,), generator=g)
        mask = (torch.arange(n)[None, :] < lengths[:, None]).float()
    elif kind == 2:  # scattered masked keys
        mask = (torch.rand(n, n, generator=g) > 0.15).float()
        if n > 3:
            mask[n // 3] = 0.0
    else:  # a fractional mask value on a band of keys
        mask[:, : max(1, n // 4)] = 0.5
        if n > 2:
            mask[-1] = 0.0
    h = 4 * 32
    weights = {
        "ln_w": 1.0 + 0.3 * torch.randn(128, generator=g),
        "ln_b": 0.2 * torch.randn(128, generator=g),
        "w_q": 0.05 * torch.randn(h, 128, generator=g),
        "w_k": 0.05 * torch.randn(h, 128, generator=g),
        "w_v": 0.05 * torch.randn(h, 128, generator=g),
        "w_g": 0.05 * torch.randn(h, 128, generator=g),
        "b_g": 0.1 * torch.randn(h, generator=g),
        "w_bias": float(torch.empty(1).uniform_(0.1, 8.0, generator=g)) * torch.randn(4, 128, generator=g) / 11.3,
        "w_o": 0.05 * torch.randn(128, h, generator=g),
        "b_o": 0.1 * torch.randn(128, generator=g),
        "eps": 1e-5,
        "inf": 1e9,
    }
    ending = bool((seed // 4) % 2)
    return n, z, mask, weights, ending, kind


@pytest.mark.parametrize("seed", range(32))
def test_random_case_meets_the_fp32_bar(seed):
    n, z, mask, w, ending, kind = _case(seed)
    print(f"seed={seed} n={n} ending={ending} masked={(mask == 0).float().mean():.3f}", flush=True)
    with torch.inference_mode():
        out = hip_block.triangle_attention_block(z.cuda(), mask.cuda(), hip_weights(w),
                                                 ending=ending)
        x_frame = (out.transpose(0, 1) if ending else out).cpu()
    mask_x = mask.transpose(0, 1) if ending else mask
    dead = (mask_x == 0).all(dim=1)  # rows whose keys are all masked
    p32 = oracle_params(w)
    p64 = p32.to(torch.float64)
    for region, sel in (("open", ~dead), ("masked", dead)):
        rows = torch.nonzero(sel).flatten()
        if rows.numel() == 0:
            continue
        ref32 = oracle.block(z, mask, p32, ending=ending, outer_rows=rows)
        ref64 = oracle.block(z.double(), mask.double(), p64, ending=ending, outer_rows=rows,
                             logits_f32=(region == "masked" or kind == 3))
        strict_close(f"seed {seed} n={n} {region}", x_frame[rows], ref64, ref32)


@pytest.mark.parametrize("seed", range(0, 32, 2))
def test_random_case_bf16_meets_the_bf16_bar(seed):
    """The same draws with BF16 storage.  Reference: the FP32 oracle on the
    same bf16-rounded inputs and weights.  Bar: max|HIP - ref| within the
    BF16 bar (2e-2 max|ref|) or twice the native BF16 path's own distance
    from ref (``oracle.block_bf16``: every intermediate rounded where the
    native path rounds it), whichever is larger -- these draws' weights give
    logits large enough that rounding them to bf16 alone moves some weights
    by percents."""
    from tests.test_gpu_bf16 import BF16_REL

    n, z, mask, w, ending, _ = _case(seed)
    print(f"bf16 seed={seed} n={n} ending={ending} masked={(mask == 0).float().mean():.3f}",
          flush=True)
    weights = hip_block.BlockWeights.from_tensors(**w, dtype=torch.bfloat16).to("cuda")
    with torch.inference_mode():
        out = hip_block.triangle_attention_block(z.to(torch.bfloat16).cuda(), mask.cuda(),
                                                 weights, ending=ending).cpu()
    assert out.dtype == torch.bfloat16 and torch.isfinite(out.float()).all()
    rounded = {k: (v.to(torch.bfloat16).float() if isinstance(v, torch.Tensor) else v)
               for k, v in w.items()}
    ref = oracle.block(z.to(torch.bfloat16).float(), mask, oracle.BlockParams(**rounded),
                       ending=ending)
    native = oracle.block_bf16(z, mask, oracle_params(w), ending=ending)
    scale = ref.abs().max().item()
    err = (out.float() - ref).abs().max().item()
    err_native = (native.float() - ref).abs().max().item()
    bar = max(BF16_REL * scale, 2.0 * err_native)
    print(f"bf16 seed {seed} n={n}: max|err| {err:.3e}, native bf16 {err_native:.3e}, "
          f"bar {bar:.3e} (max|ref| {scale:.3e})", flush=True)
    assert err <= bar


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("seed", [3, 10, 21, 28])
def test_random_case_residual_equals_z_plus_update(seed, dtype):
    """The residual entry (z += dz in place, the Pairformer's update) equals z
    plus the separate block output, rounded once in z's dtype, as the native
    z = z + tri_att(z) rounds it."""
    n, z, mask, w, ending, _ = _case(seed)
    print(f"residual seed={seed} n={n} ending={ending} dtype={dtype}", flush=True)
    weights = hip_block.BlockWeights.from_tensors(**w, dtype=dtype).to("cuda")
    with torch.inference_mode():
        zc = z.to(dtype).cuda()
        mc = mask.cuda()
        dz = hip_block.triangle_attention_block(zc, mc, weights, ending=ending)
        want = zc + dz
        hip_block.triangle_attention_block(zc, mc, weights, ending=ending, residual=True)
        assert torch.equal(zc, want), "in-place update differs from z + dz"


@pytest.mark.parametrize("n,valid,dtype", [(300, 250, torch.float32), (1536, 1352, torch.float32),
                                           (160, 140, torch.bfloat16), (1024, 900, torch.bfloat16)])
def test_repeat_calls_are_bit_identical(n, valid, dtype):
    """Padding rows with the standard weights take the constant-mask launch
    (FP32) and the BF16 block's last ring stages; both depend on counted
    waits for their LDS copies.  Eight calls on fresh workspaces, both nodes,
    must agree bit for bit."""
    print(f"repeat n={n} valid={valid} dtype={dtype}", flush=True)
    z = workloads.make_pair(n).to(dtype).cuda()
    mask = workloads.make_mask(n, valid).cuda()
    weights = hip_block.BlockWeights.from_tensors(**workloads.make_weights(bias_scale=8.0),
                                                  dtype=dtype).to("cuda")
    with torch.inference_mode():
        for ending in (False, True):
            first = hip_block.triangle_attention_block(z, mask, weights, ending=ending)
            for rep in range(7):
                again = hip_block.triangle_attention_block(z, mask, weights, ending=ending)
                assert torch.equal(first, again), f"call {rep + 1} differs (ending={ending})"
            del first, again
            torch.cuda.empty_cache()
