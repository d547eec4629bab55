"""Every entry's workspace may hold anything on entry.

The reference runs its models with
``torch.utils.deterministic.fill_uninitialized_memory = True``
(python/fireprot_workers/protenix.py:97), so an uninitialised read shows up
as a NaN there.  Here each workspace is filled with 0xFF bytes (NaN floats,
-1 integers) before the call: the result must be bit-identical to the result
on a zero-filled workspace, and the block must still meet the FP32 bar
against the float64 oracle.  Covered: the FP32 and BF16 blocks (both nodes,
with a padding tail, at sizes that do and do not fill the 128-query tiles),
the strided (OpenFold3) attention, the triangle multiplication and the pair
transition.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import block as hip_block
from fireprot_amd import openfold3 as of3
from fireprot_amd import transition as htr
from fireprot_amd import triangle_multiplication as htm
from fireprot_amd import workloads
from tests.helpers import hip_weights
from tests.test_gpu_block import _sample_rows
from tests.test_gpu_fp32_accuracy import _check_regions
from tests.test_gpu_openfold3 import make_case, qkv_view

pytestmark = pytest.mark.gpu


def _filled(nbytes: int, value: int) -> torch.Tensor:
    return torch.full((nbytes,), value, dtype=torch.uint8, device="cuda")


@pytest.mark.parametrize("n,valid", [(129, 100), (1000, 900)])
@pytest.mark.parametrize("ending", [False, True])
def test_fp32_block_on_a_poisoned_workspace(n, valid, ending):
    print(f"case fp32 block n={n} valid={valid} ending={ending}", flush=True)
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights(bias_scale=4.0)
    zc, mc, weights = z.cuda(), mask.cuda(), hip_weights(w)
    need = hip_block.workspace_bytes(n)
    outs = []
    with torch.inference_mode():
        for fill in (0xFF, 0x00):
            ws = _filled(need, fill)
            outs.append(hip_block.triangle_attention_block(zc, mc, weights, ending=ending,
                                                           workspace=ws))
            torch.cuda.synchronize()
            del ws
    poisoned, clean = outs
    assert torch.equal(poisoned, clean), "result depends on the workspace's prior contents"
    rows = torch.arange(n) if n <= 200 else _sample_rows(n, valid)
    x_frame = poisoned.transpose(0, 1) if ending else poisoned
    _check_regions(f"poisoned n={n} ending={ending}", x_frame[rows.cuda()].cpu(), z, mask, w,
                   ending, rows, valid)


@pytest.mark.parametrize("n", [129, 300])
def test_bf16_block_on_a_poisoned_workspace(n):
    z = workloads.make_pair(n).to(torch.bfloat16)
    mask = workloads.make_mask(n, n - 20)
    w = workloads.make_weights()
    zc, mc = z.cuda(), mask.cuda()
    weights = hip_block.BlockWeights.from_tensors(**w, dtype=torch.bfloat16).to("cuda")
    need = hip_block.workspace_bytes(n, torch.bfloat16)
    for ending in (False, True):
        outs = []
        with torch.inference_mode():
            for fill in (0xFF, 0x00):
                outs.append(hip_block.triangle_attention_block(
                    zc, mc, weights, ending=ending, workspace=_filled(need, fill)))
                torch.cuda.synchronize()
        assert torch.isfinite(outs[0].float()).all()
        assert torch.equal(outs[0], outs[1]), f"bf16 n={n} ending={ending}"


def test_strided_attention_on_a_poisoned_workspace():
    q, k, v, mb, bias = make_case(6, 200, 44)
    args = [qkv_view(t.cuda(), "head_last") for t in (q, k, v)]
    biases = [mb.cuda(), bias.cuda()]
    kernel = of3.StridedAttention()
    need = kernel.library.fpx_attn_strided_workspace_bytes(6, 200)
    with torch.inference_mode():
        poisoned = kernel(*args, biases, workspace=_filled(need, 0xFF))
        clean = kernel(*args, biases, workspace=_filled(need, 0x00))
        torch.cuda.synchronize()
    assert torch.equal(torch.isnan(poisoned), torch.isnan(clean))
    assert torch.equal(torch.nan_to_num(poisoned), torch.nan_to_num(clean))


@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_on_a_poisoned_workspace(outgoing):
    n = 160
    z = workloads.make_pair(n).cuda()
    mask = workloads.make_mask(n, 140).cuda()
    weights = htm.TriMulWeights.from_tensors(**workloads.make_trimul_weights()).to("cuda")
    need = htm.workspace_bytes(n)
    with torch.inference_mode():
        outs = [htm.triangle_multiplication(z, mask, weights, outgoing=outgoing,
                                            workspace=_filled(need, fill))
                for fill in (0xFF, 0x00)]
        torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])


def test_transition_on_a_poisoned_workspace():
    n = 150
    z = workloads.make_pair(n).cuda()
    weights = htr.TransitionWeights.from_tensors(**workloads.make_transition_weights()).to("cuda")
    from fireprot_amd import _native

    need = _native.library().fpx_transition_workspace_bytes(n, n, 128, 4)
    with torch.inference_mode():
        outs = [htr.transition(z, weights, workspace=_filled(need, fill)) for fill in (0xFF, 0x00)]
        torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert torch.equal(outs[0], outs[1])
