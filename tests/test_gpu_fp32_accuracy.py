"""The FP32 block computes at FP32 accuracy, held to the float64 oracle.

The reference's FP32 path is plain FP32 arithmetic (TF32 off:
python/fireprot_workers/protenix.py:113-114), and its operator tests hold the
FP32 attention core to 2e-5 against native at full N=1536
(tests/operators/test_long1536_attention.py:71).  The HIP block runs its
products on the 16-bit matrix cores through power-of-two scaled fp16 (hi, lo)
planes; these tests show that this costs no accuracy against FP32 itself.

Bar, per configuration, node and region: the HIP result's max error against
the float64 oracle must stay within max(2e-6 * max|ref|, twice the error of
the same oracle evaluated in FP32 (the native path)).  A scheme with 16-bit
significands anywhere in P.V fails it (about 6x over at C4).

Rows whose keys are all masked follow the FP32 native path's logit ties (the
-1e9 mask bias has a float32 spacing of 64), which plain float64 does not
show; their float64 reference rounds the logits to float32 at the native add
points (``logits_f32``), pinned by the brute-force fixtures.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import block as hip_block
from fireprot_amd import workloads
from oracle import triangle_attention as oracle
from tests.helpers import hip_weights, oracle_params
from tests.test_gpu_block import _sample_rows

pytestmark = pytest.mark.gpu

TOL = 2e-6


def strict_close(name: str, actual: torch.Tensor, ref64: torch.Tensor, ref32: torch.Tensor,
                 tol: float = TOL) -> None:
    """max|actual - ref64| <= max(tol * max|ref64|, 2 max|ref32 - ref64|); NaN where ref64 is."""
    actual = actual.double()
    nan = torch.isnan(ref64)
    assert torch.equal(torch.isnan(actual), nan), f"{name}: NaN positions differ"
    keep = ~nan
    err = (actual - ref64)[keep].abs().max().item() if keep.any() else 0.0
    err32 = (ref32.double() - ref64)[keep].abs().max().item() if keep.any() else 0.0
    ref = ref64[keep].abs().max().item() if keep.any() else 0.0
    bar = max(tol * ref, 2.0 * err32)
    print(f"{name}: max|err|={err:.3e} fp32 oracle {err32:.3e} max|ref|={ref:.3e} "
          f"bar={bar:.3e} ratio={err / max(err32, 1e-30):.2f}", flush=True)
    assert err <= bar, f"{name}: {err:.3e} > {bar:.3e}"


def _check_regions(name, actual, z, mask, w, ending, rows, valid):
    """actual: rows ``rows`` of the block output in the x frame."""
    p32 = oracle_params(w)
    p64 = p32.to(torch.float64)
    z64 = z.double()
    m64 = None if mask is None else mask.double()
    valid = z.shape[0] if valid is None else valid
    for region, sel in (("valid", rows < valid), ("padded", rows >= valid)):
        if not sel.any():
            continue
        sub = rows[sel]
        ref32 = oracle.block(z, mask, p32, ending=ending, outer_rows=sub)
        ref64 = oracle.block(z64, m64, p64, ending=ending, outer_rows=sub,
                             logits_f32=(region == "padded"))
        strict_close(f"{name} {region}", actual[sel], ref64, ref32)


def _run_rows(z, mask, w, ending, rows):
    with torch.inference_mode():
        out = hip_block.triangle_attention_block(
            z.cuda(), None if mask is None else mask.cuda(), hip_weights(w), ending=ending)
        x_frame = out.transpose(0, 1) if ending else out
        picked = x_frame[rows.cuda()].cpu()
        torch.cuda.synchronize()
    del out, x_frame
    torch.cuda.empty_cache()
    return picked


@pytest.mark.parametrize("ending", [False, True])
def test_c2_full_at_fp32_accuracy(ending):
    cfg = workloads.CONFIGS["c2"]
    print(f"case {cfg.name} ending={ending} (all rows)", flush=True)
    z, mask, w = workloads.make_inputs(cfg)
    rows = torch.arange(cfg.n)
    actual = _run_rows(z, mask, w, ending, rows)
    _check_regions(f"{cfg.name} ending={ending}", actual, z, mask, w, ending, rows, cfg.valid)


@pytest.mark.timeout(600)
@pytest.mark.parametrize("ending", [False, True])
def test_c3_full_at_fp32_accuracy(ending):
    """C3 (N=1000, no mask) in full: every element within the functional bar
    of the FP32 oracle (1e-4 abs + 1e-4 rel) and every row within the FP32
    bar against float64."""
    from tests.helpers import assert_f32_parity

    cfg = workloads.CONFIGS["c3"]
    print(f"case {cfg.name} ending={ending} (all rows)", flush=True)
    z, mask, w = workloads.make_inputs(cfg)
    rows = torch.arange(cfg.n)
    actual = _run_rows(z, mask, w, ending, rows)
    ref32 = oracle.block(z, mask, oracle_params(w), ending=ending)
    assert_f32_parity(f"{cfg.name} ending={ending} vs FP32 oracle",
                      actual, ref32.transpose(0, 1) if ending else ref32)
    _check_regions(f"{cfg.name} ending={ending}", actual, z, mask, w, ending, rows, cfg.valid)


@pytest.mark.parametrize("key", ["c3", "c4"])
@pytest.mark.parametrize("ending", [False, True])
def test_long_configs_sampled_rows_at_fp32_accuracy(key, ending):
    cfg = workloads.CONFIGS[key]
    rows = _sample_rows(cfg.n, cfg.valid)
    print(f"case {cfg.name} ending={ending} rows={rows.tolist()}", flush=True)
    z, mask, w = workloads.make_inputs(cfg)
    actual = _run_rows(z, mask, w, ending, rows)
    _check_regions(f"{cfg.name} ending={ending}", actual, z, mask, w, ending, rows, cfg.valid)


@pytest.mark.parametrize("bias_scale,z_scale", [(60.0, 1.0), (1e-3, 1.0), (1.0, 1e-3), (8.0, 1e3)])
def test_extreme_scales_at_fp32_accuracy(bias_scale, z_scale):
    """Logits of a few hundred, a near-zero bias, and tiny or huge z (LN
    removes the z scale up to eps): the softmax reference and the per-head
    plane scales must keep FP32 accuracy across all of them."""
    n = 200
    z = workloads.make_pair(n, z_scale)
    mask = workloads.make_mask(n, 170)
    w = workloads.make_weights(bias_scale=bias_scale)
    rows = torch.arange(n)
    for ending in (False, True):
        actual = _run_rows(z, mask, w, ending, rows)
        _check_regions(f"bias x{bias_scale} z x{z_scale} ending={ending}", actual, z, mask, w,
                       ending, rows, 170)


@pytest.mark.parametrize("v_scale", [1e-6, 1e4])
def test_value_weight_scales_at_fp32_accuracy(v_scale):
    """W_v scaled far from 1: the v^T planes' scale follows the weights'
    bound, so the products keep their accuracy relative to the values."""
    n = 160
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, 150)
    w = workloads.make_weights(bias_scale=4.0)
    w["w_v"] = w["w_v"] * v_scale
    rows = torch.arange(n)
    actual = _run_rows(z, mask, w, False, rows)
    _check_regions(f"w_v x{v_scale}", actual, z, mask, w, False, rows, 150)


def test_positive_mask_bias_rows_take_the_exact_path():
    """A mask entry of 2 gives inf * (mask - 1) = +1e9 on its key.  Such
    logits are far beyond what the fast softmax's integer reference holds
    exactly, so their rows must reproduce the native FP32 ties of
    fl(fl(s + mask) + bias) (float32 spacing 64 near 1e9), as fully masked
    rows do; the other rows keep the plain FP32 bar."""
    n = 160
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, 150)
    for i in range(0, 40):
        mask[i, (7 * i + torch.tensor([0, 11, 22])) % 30] = 2.0  # keys 0-29 only
    w = workloads.make_weights(bias_scale=4.0)
    p32 = oracle_params(w)
    p64 = p32.to(torch.float64)
    rows = torch.arange(n)
    for ending in (False, True):
        print(f"case positive mask bias ending={ending}", flush=True)
        actual = _run_rows(z, mask, w, ending, rows)
        m_x = mask.t() if ending else mask
        tied = (m_x > 1).any(1) | ~(m_x > 0).any(1)  # +1e9 keys, or every key masked
        assert tied.any() and (~tied).any()
        for region, sel in (("tied", tied), ("plain", ~tied)):
            sub = rows[sel]
            ref32 = oracle.block(z, mask, p32, ending=ending, outer_rows=sub)
            ref64 = oracle.block(z.double(), mask.double(), p64, ending=ending, outer_rows=sub,
                                 logits_f32=(region == "tied"))
            strict_close(f"positive mask ending={ending} {region}", actual[sel], ref64, ref32)


@pytest.mark.parametrize("qk_scale,inf", [(1.0, 1e9), (8.0, 1e9), (2.5, 2.0 ** 30)])
def test_padding_rows_with_and_without_the_constant_mask_shortcut(qk_scale, inf):
    """Padding rows carry one mask bias (-1e9) on every key.  While
    32 max|q| max|k| stays below half its float32 spacing (32), fl(s + m) = m
    and the attention skips S^T for them (qk_scale 1); scaling W_q and W_k by
    8 lifts |s| past that bound, so the same rows take the full exact path
    with logits spread over several float32 buckets of -1e9.  With
    inf = 2^30 the mask bias -2^30 is a power of two: its spacing is 128
    above |m| but 64 toward zero, so the bound is 32, not 64, and at
    qk_scale 2.5 (32 max|q| max|k| = 51.6 on this workload) the rows must
    take the exact path too.  All must meet the FP32 bar against float64
    with float32-rounded logits."""
    n, valid = 160, 130
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights(bias_scale=4.0)
    w["w_q"] = w["w_q"] * qk_scale
    w["w_k"] = w["w_k"] * qk_scale
    w["inf"] = inf
    rows = torch.arange(n)
    for ending in (False, True):
        print(f"case padding rows qk x{qk_scale} inf={inf:g} ending={ending}", flush=True)
        actual = _run_rows(z, mask, w, ending, rows)
        _check_regions(f"padding qk x{qk_scale} inf={inf:g} ending={ending}", actual, z, mask, w,
                       ending, rows, valid)


def test_padding_rows_with_two_mask_values():
    """Two kinds of padding rows in one block: rows 110-134 carry the mask
    bias -1e9 on every key (mask 0), rows 135-159 carry -5e8 (mask 0.5).
    The first kind has the shared weights formed once (the first constant
    row's m); chunks of four rows whose first constant row carries -5e8 take
    the per-chunk softmax; row 135, the one -5e8 row in a chunk that starts
    with -1e9 rows, takes the exact path.  W_q is scaled by 1/4 so that
    32 max|q| max|k| stays below half the float32 spacing of both mask
    biases (32 and 16).  The ending node gets the transposed mask, so its
    rows in z's transposed frame have the same kinds.  Every row meets the
    FP32 bar against float64 (float32-rounded logits on the padding rows)."""
    n, valid = 160, 110
    z = workloads.make_pair(n)
    w = workloads.make_weights(bias_scale=4.0)
    w["w_q"] = w["w_q"] * 0.25
    mask = torch.zeros(n, n)
    mask[:valid, :valid] = 1.0
    mask[135:, :] = 0.5
    rows = torch.arange(n)
    # The workspace ends with the constant-mask segment: 64 words and two
    # chunk lists (padded to 256 bytes), the weight sums [4][np], and 4 KB of
    # weight planes per (head, 32-query tile, 32-key tile).  Words 1 and 2
    # count the four-row chunks of each list: chunks 27-33 start with a -1e9
    # row, chunks 34-39 with a -5e8 row.
    np_, nkt, chunks = 256, 5, 40
    seg = lambda b: -(-b // 256) * 256  # noqa: E731
    words_at = (hip_block.workspace_bytes(n) - 4 * (np_ // 32) * nkt * 4096 - seg(4 * np_ * 4)
                - seg((64 + 2 * chunks) * 4))
    for ending in (False, True):
        m = mask.t().contiguous() if ending else mask
        print(f"case two padding mask values ending={ending}", flush=True)
        ws = torch.empty(hip_block.workspace_bytes(n), dtype=torch.uint8, device="cuda")
        with torch.inference_mode():
            out = hip_block.triangle_attention_block(z.cuda(), m.cuda(), hip_weights(w),
                                                     ending=ending, workspace=ws)
            torch.cuda.synchronize()
        x_frame = out.transpose(0, 1) if ending else out
        actual = x_frame.cpu()
        words = ws[words_at:words_at + 12].cpu().view(torch.int32)
        assert words[1].item() == 7 and words[2].item() == 6, words[:3].tolist()
        assert words[0].item() == torch.tensor([-1e9]).view(torch.int32).item()
        del out, x_frame, ws
        torch.cuda.empty_cache()
        _check_regions(f"two mask values ending={ending}", actual, z, m, w, ending, rows, valid)


def test_relative_reference_moves_for_keys_past_the_common_prefix():
    """The fast softmax starts from the relative reference C_q (the query's
    largest bias over the keys every row leaves unmasked).  Rows whose
    unmasked keys reach past that prefix can hold a far larger logit: pair
    (j, 100) of z is set along W_bias's first head, so bias[0, j, 100] is
    about 90 against a prefix maximum near 25 (bias x8), and rows with key
    100 unmasked must move their reference.  Ragged row extents (40, 60, 80
    ... 120 keys) make the common prefix one tile; both nodes meet the FP32
    bar on every row."""
    n = 160
    w = workloads.make_weights(bias_scale=8.0)
    z = workloads.make_pair(n)
    direction = w["w_bias"][0] / w["w_bias"][0].norm()
    for j in range(0, n, 7):
        z[j, 100] = 40.0 * direction
        z[100, j] = 40.0 * direction
    mask = torch.zeros(n, n)
    for i in range(n):
        mask[i, :40 + 20 * (i % 5)] = 1.0
    rows = torch.arange(n)
    p32 = oracle_params(w)
    p64 = p32.to(torch.float64)
    for ending in (False, True):
        print(f"case relative reference moves ending={ending}", flush=True)
        actual = _run_rows(z, mask, w, ending, rows)
        m_x = mask.t() if ending else mask
        dead = ~(m_x > 0).any(1)  # rows with every key masked follow the FP32 ties
        for region, sel in (("open", ~dead), ("fully masked", dead)):
            if not sel.any():
                continue
            sub = rows[sel]
            ref32 = oracle.block(z, mask, p32, ending=ending, outer_rows=sub)
            ref64 = oracle.block(z.double(), mask.double(), p64, ending=ending, outer_rows=sub,
                                 logits_f32=bool(region == "fully masked"))
            strict_close(f"relative reference ending={ending} {region}", actual[sel], ref64,
                         ref32)
