"""GPU parity of the whole block (fpx_tri_attn_block) against the CPU oracle.

Bar (FP32): max-abs 1e-4 and rel 1e-4 elementwise against the native-order
oracle on identical seeded inputs; NaN positions must agree.  Small and
medium sizes compare every element; the N=1000, N=1536 and N=4096 (the
largest the C ABI accepts) cases compare a seeded subset of outer rows (rows
are independent, so the oracle computes only those) and check
size-independent properties on the full output.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import _native
from fireprot_amd import block as hip_block
from fireprot_amd import workloads
from oracle import triangle_attention as oracle
from tests.helpers import assert_f32_parity, hip_weights, oracle_params, region_reports

pytestmark = pytest.mark.gpu


def _run(z, mask, weights, ending):
    with torch.inference_mode():
        out = hip_block.triangle_attention_block(
            z.cuda(), None if mask is None else mask.cuda(), hip_weights(weights), ending=ending)
        torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("ending", [False, True])
@pytest.mark.parametrize("n,valid", [(1, None), (5, None), (7, 5), (37, 30), (124, None),
                                     (124, 101), (129, 100), (160, None)])
def test_block_small_matches_oracle(n, valid, ending):
    print(f"case n={n} valid={valid} ending={ending}", flush=True)
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights()
    actual = _run(z, mask, w, ending)
    expected = oracle.block(z, mask, oracle_params(w), ending=ending)
    assert_f32_parity(f"n={n} valid={valid} ending={ending}", actual, expected)


def test_block_with_affine_ln_and_gate_biases():
    n = 48
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, 40)
    g = torch.Generator().manual_seed(5)
    w = workloads.make_weights()
    w["ln_w"] = 1.0 + 0.1 * torch.randn(128, generator=g)
    w["ln_b"] = 0.1 * torch.randn(128, generator=g)
    w["b_g"] = torch.randn(128, generator=g)
    w["b_o"] = 0.1 * torch.randn(128, generator=g)
    for ending in (False, True):
        actual = _run(z, mask, w, ending)
        expected = oracle.block(z, mask, oracle_params(w), ending=ending)
        assert_f32_parity(f"affine ending={ending}", actual, expected)


@pytest.mark.parametrize("ending", [False, True])
def test_c2_n512_masked_full(ending):
    cfg = workloads.CONFIGS["c2"]
    print(f"case {cfg.name} ending={ending}", flush=True)
    z, mask, w = workloads.make_inputs(cfg)
    actual = _run(z, mask, w, ending)
    expected = oracle.block(z, mask, oracle_params(w), ending=ending)
    region_reports(f"{cfg.name} ending={ending}", actual.transpose(0, 1) if ending else actual,
                   expected.transpose(0, 1) if ending else expected, cfg.valid)
    assert_f32_parity(f"{cfg.name} ending={ending}", actual, expected)


def _sample_rows(n, valid, count=12, seed=11):
    g = torch.Generator().manual_seed(seed)
    rows = {0, 1, n - 1, n // 2}
    if valid is not None and valid < n:
        rows |= {valid - 1, valid, min(valid + 1, n - 1)}
    rows |= set(torch.randint(0, n, (count,), generator=g).tolist())
    return torch.tensor(sorted(rows))


@pytest.mark.parametrize("key", ["c3", "c4"])
def test_long_configs_row_subset_and_transpose_identity(key):
    cfg = workloads.CONFIGS[key]
    print(f"case {cfg.name}", flush=True)
    z, mask, w = workloads.make_inputs(cfg)
    params = oracle_params(w)
    rows = _sample_rows(cfg.n, cfg.valid)
    zc = z.cuda()
    mc = None if mask is None else mask.cuda()
    weights = hip_weights(w)
    with torch.inference_mode():
        start = hip_block.triangle_attention_block(zc, mc, weights, ending=False)
        end = hip_block.triangle_attention_block(zc, mc, weights, ending=True)
        # ending node == T(starting node on T(z), T(mask)), bit for bit
        zt = zc.transpose(0, 1).contiguous()
        mt = None if mc is None else mc.transpose(0, 1).contiguous()
        end_ref = hip_block.triangle_attention_block(zt, mt, weights, ending=False).transpose(0, 1)
        again = hip_block.triangle_attention_block(zc, mc, weights, ending=False)
        torch.cuda.synchronize()
        assert torch.equal(end, end_ref), "ending node differs from T(start(T(z)))"
        assert torch.equal(start, again), "block is not deterministic"
        assert torch.isfinite(start).all() and torch.isfinite(end).all()
        start_rows = start[rows.cuda()].cpu()
        end_rows = end.transpose(0, 1)[rows.cuda()].cpu()
    del zc, zt, start, end, end_ref, again
    torch.cuda.empty_cache()
    exp_start = oracle.block(z, mask, params, ending=False, outer_rows=rows)
    exp_end = oracle.block(z, mask, params, ending=True, outer_rows=rows)
    region_reports(f"{cfg.name} start", start_rows, exp_start, cfg.valid, rows)
    region_reports(f"{cfg.name} end", end_rows, exp_end, cfg.valid, rows)
    assert_f32_parity(f"{cfg.name} start rows", start_rows, exp_start)
    assert_f32_parity(f"{cfg.name} end rows", end_rows, exp_end)


@pytest.mark.timeout(600)
def test_maximum_n4096_row_subset_and_transpose_identity():
    """The largest pair size the C ABI accepts (N = 4096: 128 key tiles, the
    tile-flag words full, [N][N][128] tensors of 2^31 elements), with a
    padding tail of 296 residues; both nodes on a few outer rows against the
    oracle, and the ending node equal to T(start(T(z))) bit for bit.  z is
    drawn on the GPU (a seeded device generator) and copied to the host for
    the oracle."""
    n, valid = 4096, 3800
    print(f"case maximum n={n} valid={valid}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(419 + n)
    zc = torch.randn(n, n, 128, generator=g, device="cuda")
    mc = workloads.make_mask(n, valid).cuda()
    w = workloads.make_weights()
    weights = hip_weights(w)
    gr = torch.Generator().manual_seed(n)
    rows = torch.tensor(sorted({0, valid - 1, valid, n - 1,
                                int(torch.randint(0, valid, (1,), generator=gr))}))
    with torch.inference_mode():
        start = hip_block.triangle_attention_block(zc, mc, weights, ending=False)
        end = hip_block.triangle_attention_block(zc, mc, weights, ending=True)
        start_rows = start[rows.cuda()].cpu()
        end_rows = end.transpose(0, 1)[rows.cuda()].cpu()
        assert torch.isfinite(start).all() and torch.isfinite(end).all()
        del start
        zt = zc.transpose(0, 1).contiguous()
        end_ref = hip_block.triangle_attention_block(zt, mc.t().contiguous(), weights,
                                                     ending=False).transpose(0, 1)
        torch.cuda.synchronize()
        assert torch.equal(end, end_ref), "ending node differs from T(start(T(z)))"
    z = zc.cpu()
    mask = mc.cpu()
    del zc, zt, end, end_ref
    torch.cuda.empty_cache()
    params = oracle_params(w)
    exp_start = oracle.block(z, mask, params, ending=False, outer_rows=rows)
    exp_end = oracle.block(z, mask, params, ending=True, outer_rows=rows)
    region_reports(f"n={n} start", start_rows, exp_start, valid, rows)
    region_reports(f"n={n} end", end_rows, exp_end, valid, rows)
    assert_f32_parity(f"n={n} start rows", start_rows, exp_start)
    assert_f32_parity(f"n={n} end rows", end_rows, exp_end)


@pytest.mark.parametrize("ending", [False, True])
def test_block_large_bias_scale(ending):
    """Triangle-bias weights x60: logits of a few hundred, far outside the
    range where the kernel's softmax reference stays at 0."""
    n = 200
    z = workloads.make_pair(n)
    w = workloads.make_weights(bias_scale=60.0)
    actual = _run(z, None, w, ending)
    expected = oracle.block(z, None, oracle_params(w), ending=ending)
    assert_f32_parity(f"bias x60 ending={ending}", actual, expected)


def _end_weights(w):
    """A second weight set for the ending node (rows rolled, bias rescaled)."""
    out = {k: (None if v is None else torch.roll(v, 7, 0).contiguous()) for k, v in w.items()}
    out["w_bias"] = out["w_bias"] * 1.5
    return out


@pytest.mark.parametrize("n,valid", [(124, 101), (200, None)])
def test_pair_step_residual_in_place(n, valid):
    """z += tri_att_start(z); z += tri_att_end(z) in place, as the Pairformer
    step does it (patches/protenix/0006-*.patch:17-37)."""
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    ws, we = workloads.make_weights(), _end_weights(workloads.make_weights())
    z1 = z + oracle.block(z, mask, oracle_params(ws), ending=False)
    expected = z1 + oracle.block(z1, mask, oracle_params(we), ending=True)
    zc = z.cuda()
    with torch.inference_mode():
        out = hip_block.pair_step_triangle_attention(
            zc, None if mask is None else mask.cuda(), hip_weights(ws), hip_weights(we))
        torch.cuda.synchronize()
    assert out.data_ptr() == zc.data_ptr()
    assert_f32_parity(f"pair step n={n}", zc.cpu(), expected)


def test_residual_into_separate_buffer_and_alias_guard():
    n = 64
    z, mask, w = workloads.make_pair(n), workloads.make_mask(n, 50), workloads.make_weights()
    base = torch.randn(n, n, 128, generator=torch.Generator().manual_seed(3))
    expected = base + oracle.block(z, mask, oracle_params(w), ending=True)
    out = base.cuda()
    zc = z.cuda()
    with torch.inference_mode():
        hip_block.triangle_attention_block(zc, mask.cuda(), hip_weights(w), ending=True, out=out,
                                           residual=True)
        torch.cuda.synchronize()
    assert torch.equal(zc.cpu(), z)
    assert_f32_parity("residual into out", out.cpu(), expected)
    # z_out == z with different strides is rejected before any launch
    lib = _native.library()
    wt = hip_weights(w)
    ws = torch.empty(hip_block.workspace_bytes(n), dtype=torch.uint8, device="cuda")
    code = lib.fpx_tri_attn_block_residual(
        0, zc.data_ptr(), zc.stride(0), zc.stride(1), None, 0, 0, None, None, 1e-5,
        wt.w_qkvg.data_ptr(), None, wt.w_bias.data_ptr(), wt.w_o.data_ptr(), None, 1e9,
        n, 128, 4, 32, 0, zc.data_ptr(), zc.stride(1), zc.stride(0), ws.data_ptr(), ws.numel(),
        torch.cuda.current_stream().cuda_stream)
    assert code == 2


def test_block_inputs_unchanged_streams_and_queue():
    n = 96
    z, mask, w = workloads.make_pair(n), workloads.make_mask(n, 80), workloads.make_weights()
    expected = oracle.block(z, mask, oracle_params(w), ending=False)
    zc, mc, weights = z.cuda(), mask.cuda(), hip_weights(w)
    saved = [t.clone() for t in (zc, mc, weights.w_qkvg, weights.w_bias, weights.w_o)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode(), torch.cuda.stream(stream):
        outs = [hip_block.triangle_attention_block(zc, mc, weights) for _ in range(3)]
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for out in outs:
        assert out.is_contiguous()
        assert_f32_parity("queued", out.cpu(), expected)
    for t, before in zip((zc, mc, weights.w_qkvg, weights.w_bias, weights.w_o), saved):
        assert torch.equal(t, before)


def test_block_output_canaries_and_strided_dz():
    n = 64
    z, mask, w = workloads.make_pair(n), workloads.make_mask(n, 50), workloads.make_weights()
    expected = oracle.block(z, mask, oracle_params(w), ending=True)
    storage = torch.full((n * n * 128 + 8192,), 123.5, device="cuda")
    out = storage[4096:-4096].view(n, n, 128)
    with torch.inference_mode():
        hip_block.triangle_attention_block(z.cuda(), mask.cuda(), hip_weights(w), ending=True,
                                           out=out)
        torch.cuda.synchronize()
    assert bool((storage[:4096] == 123.5).all()) and bool((storage[-4096:] == 123.5).all())
    assert_f32_parity("canary", out.cpu(), expected)


@pytest.mark.parametrize("name", ["n5_plain", "n7_tail", "n9_random_x8", "n6_order"])
@pytest.mark.parametrize("ending", [False, True])
def test_block_matches_golden_fixtures(name, ending):
    """The HIP block against the brute-force fixtures' FP32-logit expectation,
    fully masked rows included (their -1e9-quantised ties must match)."""
    from tests.test_oracle import load_case

    z, mask, params, expected = load_case(name, torch.float32)
    weights = {k: getattr(params, k) for k in ("ln_w", "ln_b", "w_q", "w_k", "w_v", "w_g",
                                                "b_g", "w_bias", "w_o", "b_o")}
    actual = _run(z, mask, weights, ending)
    tag = "end" if ending else "start"
    torch.testing.assert_close(actual.double(), expected[f"dz_{tag}_f32l"], atol=2e-6, rtol=1e-4)
