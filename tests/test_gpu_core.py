"""GPU parity of the attention core (fpx_attn_core / fpx_attn_core_masked) and
of the operator-level dispatch, against the oracle's native ``_attention``.

Mirrors the reference's adversarial set (tests/operators/test_ck_attention*.py):
-inf bias rows and a +80 key, masked keys, non-contiguous head-last inputs,
input immutability, non-default streams, queued calls, output canaries and
the C-ABI guard codes.  A fully -inf row yields NaN, as torch.softmax does.
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import _native
from fireprot_amd import triangle_attention as ta
from fireprot_amd.registry import registry
from oracle import triangle_attention as oracle
from tests.helpers import assert_f32_parity

pytestmark = pytest.mark.gpu


def _inputs(batch, n, seed, *, masked=False):
    g = torch.Generator().manual_seed(seed)
    q, k, v = [torch.randn(batch, n, 4, 32, generator=g).transpose(1, 2) for _ in range(3)]
    q = q / 32 ** 0.5
    bias = torch.randn(n, n, 4, generator=g).permute(2, 0, 1).unsqueeze(0)
    biases = [bias]
    if masked:
        keep = torch.randint(0, 2, (batch, 1, 1, n), generator=g).float()
        keep[..., 0] = 1.0
        biases.insert(0, 1e9 * (keep - 1))
    return q, k, v, biases


def _expected(q, k, v, biases):
    return oracle.attention_core(q, k, v, [b.clone() for b in biases]).transpose(-2, -3)


def _cuda(q, k, v, biases):
    # keep the head-last projection layout: [B, N, H, D] memory viewed as [B, H, N, D]
    def dev(t):
        return t.transpose(1, 2).contiguous().cuda().transpose(1, 2)
    return dev(q), dev(k), dev(v), [b.cuda() for b in biases]


@pytest.mark.parametrize("batch,n,masked", [(3, 4, False), (5, 20, True), (4, 124, False),
                                            (4, 124, True), (2, 1000, False), (2, 1000, True),
                                            (2, 1536, False), (1, 132, True), (2, 1536, True)])
def test_core_matches_native(batch, n, masked):
    print(f"case core batch={batch} n={n} masked={masked}", flush=True)
    q, k, v, biases = _inputs(batch, n, 100 + n, masked=masked)
    expected = _expected(q, k, v, biases)
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    registry.clear_runtime_state()
    with torch.inference_mode():
        actual = ta.dispatch_triangle_attention(
            module=SimpleNamespace(training=False), q=qc, k=kc, v=vc, biases=bc,
            native=lambda **_: pytest.fail("native selected"))
        torch.cuda.synchronize()
    assert actual.shape == (batch, n, 4, 32) and actual.is_contiguous()
    assert_f32_parity(f"core b={batch} n={n} masked={masked}", actual.cpu(), expected)
    assert registry.count(ta.OPERATION, ta.IMPLEMENTATION) == 1


def test_core_extreme_bias_rows_and_inputs_unchanged():
    q, k, v, biases = _inputs(3, 64, 7)
    bias = biases[0].clone()
    bias[:, :, 0, :] = float("-inf")   # all -inf query row -> NaN (torch.softmax)
    bias[:, :, 1, 0] = 80.0            # one dominant key
    bias[:, :, 2, :40] = float("-inf")  # leading -inf tiles, finite later
    biases = [bias]
    expected = _expected(q, k, v, biases)
    assert torch.isnan(expected[:, 0]).all() and torch.isfinite(expected[:, 1:]).all()
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    saved = [t.clone() for t in (qc, kc, vc, bc[0])]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode(), torch.cuda.stream(stream):
        outs = [ta.attention(module=None, q=qc, k=kc, v=vc, biases=bc, native=None)
                for _ in range(3)]
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for out in outs:
        assert_f32_parity("extreme", out.cpu(), expected)
    for t, before in zip((qc, kc, vc, bc[0]), saved):
        assert torch.equal(t, before)


def test_core_reference_regimes():
    """Rows that drive every branch of the kernel's softmax reference: a large
    positive and a large negative row max (reference away from 0), a row
    whose running sum passes 2^64 without any single weight doing so, a late
    +200 key, and leading -inf tiles, side by side in one wavefront."""
    batch, n = 2, 1000
    q, k, v, biases = _inputs(batch, n, 31)
    g = torch.Generator().manual_seed(32)
    bias = biases[0].clone()
    noise = torch.randn(4, n, generator=g)
    bias[0, :, 0, :] = 300.0 + noise          # log2 logits ~433: reference c = max
    bias[0, :, 1, :32] = 30.0                  # first tile ~43 (log2): c snaps to 0 ...
    bias[0, :, 1, 32:] = 38.5                  # ... then 968 keys at ~55.5 push the sum past 2^64
    bias[0, :, 2, :] = noise
    bias[0, :, 2, 700] = 200.0                 # a late dominant key
    bias[0, :, 3, :] = -300.0 + noise          # large negative row
    bias[0, :, 4, :96] = float("-inf")         # three leading -inf tiles
    bias[0, :, 33, :] = 150.0 + noise          # second wavefront: large row
    biases = [bias]
    expected = _expected(q, k, v, biases)
    assert torch.isfinite(expected).all()
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    with torch.inference_mode():
        out = ta.attention(module=None, q=qc, k=kc, v=vc, biases=bc, native=None)
        torch.cuda.synchronize()
    assert_f32_parity("reference regimes", out.cpu(), expected)


def test_core_c_abi_guards_and_canaries():
    lib = _native.library()
    # invalid sizes are rejected before any pointer is dereferenced
    assert lib.fpx_attn_core(None, None, None, None, None, 1, 6, None) == 2
    assert lib.fpx_attn_core(None, None, None, None, None, 0, 8, None) == 2
    assert lib.fpx_attn_core(None, None, None, None, None, 1, 8, None) == 3
    assert lib.fpx_attn_core(4, 16, 16, 16, 16, 1, 8, None) == 3
    q, k, v, biases = _inputs(2, 100, 9)
    expected = _expected(q, k, v, biases)
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    bias = bc[0].contiguous()
    storage = torch.full((qc.numel() + 8192,), 123.5, device="cuda")
    out = storage[4096:-4096]
    code = lib.fpx_attn_core(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), bias.data_ptr(),
                             out.data_ptr(), 2, 100, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert code == 0
    assert_f32_parity("canary core", out.view(2, 100, 4, 32).cpu(), expected)
    assert bool((storage[:4096] == 123.5).all()) and bool((storage[-4096:] == 123.5).all())


def test_core_padded_bias_row_stride():
    """A 1552-float bias row stride at N=1536, as the reference pads it."""
    q, k, v, biases = _inputs(1, 1536, 21)
    expected = _expected(q, k, v, biases)
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    padded = torch.zeros((1, 4, 1536, 1552), device="cuda")
    padded[..., :1536].copy_(bc[0])
    out = torch.empty((1, 1536, 4, 32), device="cuda")
    lib = _native.library()
    code = lib.fpx_attn_core_masked(qc.data_ptr(), kc.data_ptr(), vc.data_ptr(), None, 0,
                                    padded.data_ptr(), 1552, out.data_ptr(), 1, 1536,
                                    torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert code == 0
    assert_f32_parity("padded stride", out.cpu(), expected)


def test_dispatch_falls_back_for_unsupported_shapes():
    """Three heads of dimension 32 (the projection layout of another model):
    the candidate rejects the shape with a reason and native runs."""
    g = torch.Generator().manual_seed(3)
    q, k, v = [torch.randn(2, 6, 3, 32, generator=g).transpose(1, 2).cuda() for _ in range(3)]
    bias = torch.randn(1, 3, 6, 6, generator=g).cuda()
    registry.clear_runtime_state()
    with torch.inference_mode():
        result = ta.dispatch_triangle_attention(module=SimpleNamespace(training=False), q=q,
                                                k=k, v=v, biases=[bias],
                                                native=lambda **_: "native")
    assert result == "native"
    decision = registry.manifest()["decisions"][0]
    assert decision["selected"] == "native"
    assert "4 heads of dimension 32" in decision["rejected"][0]["reason"]


@pytest.mark.parametrize("batch,n,masked", [(2, 6, False), (3, 129, True), (1, 1, False)])
def test_dispatch_serves_any_sequence_length(batch, n, masked):
    """The plane-staged route takes any N up to 4096 (N % 4 != 0 included):
    the candidate is selected and meets the FP32 functional bar."""
    print(f"case core any n batch={batch} n={n} masked={masked}", flush=True)
    q, k, v, biases = _inputs(batch, n, 200 + n, masked=masked)
    expected = _expected(q, k, v, biases)
    qc, kc, vc, bc = _cuda(q, k, v, biases)
    registry.clear_runtime_state()
    with torch.inference_mode():
        actual = ta.dispatch_triangle_attention(
            module=SimpleNamespace(training=False), q=qc, k=kc, v=vc, biases=bc,
            native=lambda **_: pytest.fail("native selected"))
        torch.cuda.synchronize()
    assert_f32_parity(f"core any n b={batch} n={n}", actual.cpu(), expected)
    assert registry.count(ta.OPERATION, ta.IMPLEMENTATION) == 1
