"""The exact bf16 plane split behind every FP32-accurate kernel, bit for bit.

Every product of the block, the triangle multiplication and the transition
runs on the BF16 matrix cores over operands split as hi = bf16(x),
lo = bf16(x - hi), rest = bf16(x - hi - lo) (round to nearest even), with
hi + lo + rest == x for normal x.  ``fpx_split_planes`` runs the device split
the kernels use; the expected planes here come from integer bit arithmetic
and float64 differences on the host, which are exact.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from fireprot_amd import _native

pytestmark = pytest.mark.gpu


def bf16_rne_bits(x: np.ndarray) -> np.ndarray:
    """Round float32 values to bfloat16 (nearest, ties to even); the 16 bits."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    bias = 0x7FFF + ((u >> 16) & 1)
    return ((u + bias) >> 16).astype(np.uint16)


def bf16_value(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def inputs(count: int) -> np.ndarray:
    rng = np.random.default_rng(1187)
    x = rng.standard_normal(count) * np.exp2(rng.integers(-90, 90, count))
    x = x.astype(np.float32)
    # exact bf16 values (lo = rest = 0), zeros of both signs, and ties: a
    # bf16 value plus exactly half its last place (rounds to the even one)
    x[:8] = [0.0, -0.0, 1.0, -2.5, 3.0e38, -1.0e-30, 65504.0, 1.0 / 3.0]
    base = bf16_value(bf16_rne_bits(x[8:64]))
    _, exponent = np.frexp(base)  # |base| in [2^(e-1), 2^e): bf16 ulp 2^(e-8)
    x[8:64] = (base + np.sign(base) * np.exp2(exponent - 9.0)).astype(np.float32)
    # values whose residual after hi needs all 24 bits
    x[64:128] = (1.0 + np.arange(64, dtype=np.float32) * np.float32(2.0 ** -23)) * np.float32(7.0)
    return x


def run_split(x: np.ndarray) -> np.ndarray:
    lib = _native.library()
    xc = torch.from_numpy(x).cuda()
    planes = torch.zeros(5, x.size, dtype=torch.int16, device="cuda")
    code = lib.fpx_split_planes(xc.data_ptr(), x.size, planes.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_split_planes")
    torch.cuda.synchronize()
    return planes.cpu().numpy().view(np.uint16)


def test_three_plane_split_is_exact_and_round_to_nearest_even():
    x = inputs(1 << 16)
    planes = run_split(x)
    hi_bits = bf16_rne_bits(x)
    hi = bf16_value(hi_bits)
    r1 = x.astype(np.float64) - hi
    assert np.all(r1.astype(np.float32).astype(np.float64) == r1), "x - hi not exact in fp32"
    lo_bits = bf16_rne_bits(r1.astype(np.float32))
    lo = bf16_value(lo_bits)
    r2 = r1 - lo
    rest_bits = bf16_rne_bits(r2.astype(np.float32))
    np.testing.assert_array_equal(planes[0], hi_bits)
    np.testing.assert_array_equal(planes[1], lo_bits)
    np.testing.assert_array_equal(planes[2], rest_bits)
    total = bf16_value(planes[0]) + bf16_value(planes[1]) + bf16_value(planes[2])
    finite = np.abs(x) < 3.0e38  # the 3e38 entry rounds hi to inf in bf16
    np.testing.assert_array_equal(total[finite], x.astype(np.float64)[finite])


def test_two_plane_split_matches_the_first_two_planes():
    x = inputs(1 << 14)
    planes = run_split(x)
    np.testing.assert_array_equal(planes[3], planes[0])
    np.testing.assert_array_equal(planes[4], planes[1])


def test_split_rejects_ragged_counts():
    lib = _native.library()
    x = torch.zeros(12, device="cuda")
    out = torch.zeros(5, 16, dtype=torch.int16, device="cuda")
    assert lib.fpx_split_planes(x.data_ptr(), 12, out.data_ptr(), None) == _native.FPX_ERR_DIMS
    assert lib.fpx_split_planes(x.data_ptr() + 4, 8, out.data_ptr(), None) == _native.FPX_ERR_POINTER
