"""fpx_tri_attn_block_noalloc: the block with the library's own fixed
scratch array instead of a caller workspace.

Called through the C ABI twice in a row on one GPU, the second call with a
smaller pair size, each result must be bit-identical to fpx_tri_attn_block's
on a caller workspace (the same kernels on the same inputs), for the FP32 and
the BF16 block and both nodes.  Sizes past the array's maximum (N > 128) are
refused with status 2 before any launch.  The no-allocation entry shares one
array per GPU, so the calls here run one after another on one stream.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import _native
from fireprot_amd import block as hip_block
from fireprot_amd import workloads

pytestmark = pytest.mark.gpu


def _args(z, mask, weights, ending, out):
    ptr = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    return (hip_block.DTYPES[z.dtype], z.data_ptr(), z.stride(0), z.stride(1),
            ptr(mask), mask.stride(0) if mask is not None else 0,
            mask.stride(1) if mask is not None else 0,
            ptr(weights.ln_w), ptr(weights.ln_b), weights.eps, weights.w_qkvg.data_ptr(),
            ptr(weights.b_g), weights.w_bias.data_ptr(), weights.w_o.data_ptr(),
            ptr(weights.b_o), weights.inf, z.shape[0], 128, 4, 32, int(ending),
            out.data_ptr(), out.stride(0), out.stride(1))


def _both(lib, z, mask, weights, ending):
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.empty_like(z)
    ws = torch.empty(hip_block.workspace_bytes(z.shape[0], z.dtype), dtype=torch.uint8,
                     device="cuda")
    _native.check(lib.fpx_tri_attn_block(*_args(z, mask, weights, ending, ref), ws.data_ptr(),
                                         ws.numel(), stream), "fpx_tri_attn_block")
    got = torch.full_like(z, float("nan"))
    _native.check(lib.fpx_tri_attn_block_noalloc(*_args(z, mask, weights, ending, got), stream),
                  "fpx_tri_attn_block_noalloc")
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_block_matches_the_workspace_entry_on_consecutive_calls(dtype):
    lib = _native.library()
    w = workloads.make_weights(bias_scale=4.0)
    weights = hip_block.BlockWeights.from_tensors(**w, dtype=dtype).to("cuda")
    with torch.inference_mode():
        for n, valid in ((128, 110), (61, 50)):  # the second call is smaller
            z = workloads.make_pair(n).to(dtype).cuda()
            mask = workloads.make_mask(n, valid).cuda()
            for ending in (False, True):
                ref, got = _both(lib, z, mask, weights, ending)
                print(f"noalloc {dtype} n={n} ending={ending}", flush=True)
                assert torch.isfinite(ref.float()).all()
                assert torch.equal(got, ref), f"{dtype} n={n} ending={ending}"


def test_noalloc_block_refuses_sizes_past_its_array():
    lib = _native.library()
    w = hip_block.BlockWeights.from_tensors(**workloads.make_weights()).to("cuda")
    z = workloads.make_pair(129).cuda()
    out = torch.zeros_like(z)
    code = lib.fpx_tri_attn_block_noalloc(*_args(z, None, w, False, out),
                                          torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert code == _native.FPX_ERR_DIMS
    assert bool((out == 0).all()), "nothing may run for a refused size"
