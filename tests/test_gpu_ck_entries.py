"""The reference's three attention entries, bound and called as it does.

python/fireprot/backends/amd/ck_attention.py:65-73 binds ``ck_attention``,
``ck_attention_exact1536`` and ``ck_attention_vector_bias1000`` from one
library with argtypes ``[c_void_p] * 5 + [c_int] * 2 + [c_void_p]`` and
restype ``c_int``; its ``attention()`` (ck_attention.py:115-141) picks the
exact-1536 entry at N=1536 and the vector-bias entry at N=1000, copies the
bias into ``[1, 4, 1536, 1552]`` rows at N=1536, allocates the output with
``empty_like(q)``, calls the entry on the current stream and returns
``output.transpose(-2, -3)``.  These tests follow that sequence against this
library's exports, at the two shapes the reference serves (B512 N1536, B1000
N1000), and compare sampled batch rows with the float64 oracle at the FP32
bar of tests/test_gpu_fp32_accuracy.py.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

from fireprot_amd import _native
from oracle import triangle_attention as oracle
from tests.test_gpu_fp32_accuracy import strict_close

pytestmark = pytest.mark.gpu


def _bound(name: str):
    """The entry as the reference's loader binds it (its own argtypes)."""
    fn = getattr(ctypes.CDLL(str(_native.LIB_PATH)), name)
    fn.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 2 + [ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


def _operands(batch: int, n: int, seed: int):
    """q, k, v as [B, 4, N, 32] views of head-last [B, N, 4, 32] memory (the
    projection layout, strides (N*128, 32, 128, 1)), q scaled by 1/sqrt(32);
    the triangle bias [1, 4, N, N] (std 8: logits of +-40)."""
    g = torch.Generator(device="cuda").manual_seed(seed)

    def head_last():
        return torch.randn(batch, n, 4, 32, generator=g, device="cuda").transpose(1, 2)

    q = head_last() / 32 ** 0.5
    k, v = head_last(), head_last()
    bias = 8.0 * torch.randn(1, 4, n, n, generator=g, device="cuda")
    return q, k, v, bias


def _reference_call(entry, q, k, v, biases):
    """The body of the reference's attention() after it picked ``entry``."""
    with torch.cuda.device(q.device):
        if q.shape[2] == 1536:
            bias = torch.empty((1, 4, 1536, 1552), device=q.device, dtype=q.dtype)
            bias[..., :1536].copy_(biases[0])
        else:
            bias = biases[0].contiguous()
        output = torch.empty_like(q)
        status = entry(q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.data_ptr(),
                       output.data_ptr(), q.shape[0], q.shape[2],
                       torch.cuda.current_stream(q.device).cuda_stream)
        if status:
            raise RuntimeError(f"attention launch failed with status {status}")
    return output.transpose(-2, -3)


def _check_rows(name, out, q, k, v, bias, rows):
    """out: [B, 4, N, 32], the layout of q."""
    qs, ks, vs = (t[rows].cpu() for t in (q, k, v))
    b = bias.cpu()
    ref64 = oracle.attention_core(qs.double(), ks.double(), vs.double(), [b.double()])
    ref32 = oracle.attention_core(qs, ks, vs, [b.clone()])
    strict_close(name, out[rows].cpu(), ref64, ref32)


@pytest.mark.parametrize("entry_name,batch,n", [("ck_attention_exact1536", 512, 1536),
                                                ("ck_attention", 512, 1536),
                                                ("ck_attention_vector_bias1000", 1000, 1000),
                                                ("ck_attention", 1000, 1000)])
def test_reference_attention_flow(entry_name, batch, n):
    print(f"case {entry_name} batch={batch} n={n}", flush=True)
    q, k, v, bias = _operands(batch, n, 900 + n)
    entry = _bound(entry_name)
    saved = [t.clone() for t in (q, k, v, bias)]
    with torch.inference_mode():
        out = _reference_call(entry, q, k, v, [bias])
        torch.cuda.synchronize()
    assert out.shape == (batch, n, 4, 32)
    for t, before in zip((q, k, v, bias), saved):
        assert torch.equal(t, before), "inputs must not change"
    rows = torch.tensor([0, 1, batch // 2, batch - 1])
    _check_rows(f"{entry_name} b={batch} n={n}", out.transpose(-2, -3), q, k, v, bias, rows)


def test_fpx_attn_core_reads_a_contiguous_bias_at_1536():
    """fpx_attn_core reads a contiguous [1, 4, N, N] bias at every N, N=1536
    included, for a batch the reference entries do not accept (the padded
    1552-float rows are the ck_attention* entries' convention only)."""
    batch, n = 3, 1536
    q, k, v, bias = _operands(batch, n, 77)
    entry = _bound("fpx_attn_core")
    with torch.inference_mode():
        output = torch.empty_like(q)
        status = entry(q.data_ptr(), k.data_ptr(), v.data_ptr(), bias.contiguous().data_ptr(),
                       output.data_ptr(), batch, n, torch.cuda.current_stream().cuda_stream)
        assert status == 0, status
        out = output.transpose(-2, -3)
        torch.cuda.synchronize()
    _check_rows("fpx_attn_core b=3 n=1536", out.transpose(-2, -3), q, k, v, bias,
                torch.arange(batch))
