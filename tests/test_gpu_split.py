"""The fp16 (hi, lo) split behind every FP32-accurate product, bit for bit.

Every product of the FP32 block, the triangle multiplication and the
transition runs on the 16-bit matrix cores over operands scaled by a power of
two per block and split as hi = fp16(x), lo = fp16(x - hi) (round to nearest
even; x - hi is exact in FP32).  The device forms hi with v_cvt_pk_f16_f32,
the residual with one v_fma_mix_f32 per value and lo with one more
v_cvt_pk_f16_f32 per pair.  ``fpx_split_planes`` runs that
device split; the expected planes here come from numpy's float16 conversion
of the value and of its exact float32 residual.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from fireprot_amd import _native

pytestmark = pytest.mark.gpu


def inputs(count: int) -> np.ndarray:
    rng = np.random.default_rng(1187)
    x = rng.standard_normal(count) * np.exp2(rng.integers(-30, 18, count))
    x = x.astype(np.float32)
    # exact fp16 values (lo = 0), zeros of both signs, the range ends and
    # non-finite values
    x[:16] = [0.0, -0.0, 1.0, -2.5, 65504.0, -65504.0, 65519.0, 65520.0,
              np.inf, -np.inf, np.nan, 6.1035156e-05, 5.9604645e-08, -1.0e-9, 16384.0, 1.0 / 3.0]
    # ties: an fp16 value plus exactly half its last place (rounds to the even one)
    base = rng.uniform(1.0, 30000.0, 48).astype(np.float16).astype(np.float64)
    _, exponent = np.frexp(base)  # base in [2^(e-1), 2^e): fp16 ulp 2^(e-11)
    x[16:64] = (base + np.exp2(exponent - 12.0)).astype(np.float32)
    # values whose residual after hi needs all 24 bits
    x[64:128] = (1.0 + np.arange(64, dtype=np.float32) * np.float32(2.0 ** -23)) * np.float32(7.0)
    return x


def expected(x: np.ndarray):
    with np.errstate(over="ignore", invalid="ignore"):
        hi = x.astype(np.float16)
        residual = (x.astype(np.float64) - hi.astype(np.float64)).astype(np.float32)
        lo = residual.astype(np.float16)
    return hi, lo


def run_split(x: np.ndarray) -> np.ndarray:
    lib = _native.library()
    xc = torch.from_numpy(x).cuda()
    planes = torch.zeros(2, x.size, dtype=torch.int16, device="cuda")
    code = lib.fpx_split_planes(xc.data_ptr(), x.size, planes.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_split_planes")
    torch.cuda.synchronize()
    return planes.cpu().numpy().view(np.float16)


def test_fp16_split_matches_round_to_nearest_even_bit_for_bit():
    x = inputs(1 << 16)
    hi, lo = run_split(x)
    want_hi, want_lo = expected(x)
    for got, want, name in ((hi, want_hi, "hi"), (lo, want_lo, "lo")):
        nan = np.isnan(want)
        np.testing.assert_array_equal(np.isnan(got), nan, err_msg=f"{name}: NaN positions")
        np.testing.assert_array_equal(got[~nan].view(np.uint16), want[~nan].view(np.uint16),
                                      err_msg=f"{name} bits")


def test_two_planes_hold_22_bits_in_the_scaled_range():
    x = inputs(1 << 14)
    hi, lo = run_split(x)
    ax = np.abs(x.astype(np.float64))
    sel = (ax >= 0.25) & (ax <= 65504.0)
    with np.errstate(invalid="ignore"):  # inf + -inf outside the selected range
        total = hi.astype(np.float64) + lo.astype(np.float64)
    err = np.abs(total[sel] - x.astype(np.float64)[sel]) / ax[sel]
    assert err.max() <= 2.0 ** -22, err.max()


def test_split_rejects_ragged_counts():
    lib = _native.library()
    x = torch.zeros(12, device="cuda")
    out = torch.zeros(2, 16, dtype=torch.int16, device="cuda")
    assert lib.fpx_split_planes(x.data_ptr(), 12, out.data_ptr(), None) == _native.FPX_ERR_DIMS
    assert lib.fpx_split_planes(x.data_ptr() + 4, 8, out.data_ptr(), None) == _native.FPX_ERR_POINTER
