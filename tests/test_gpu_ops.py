"""GPU parity of the stage kernels: LayerNorm (contiguous and transposed view),
the fused q/k/v projection and the sigmoid gate, against the oracle's native
ops.  Mirrors tests/operators/test_transposed_norm.py (stress rows),
test_qkv_projection.py (layout strides, extreme rows) and
test_attention_gate.py (linspace(-1000, 1000) gate) of the reference.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import attention_gate, layer_norm, qkv_projection
from oracle import triangle_attention as oracle
from tests.helpers import assert_f32_parity

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("n", [124, 1000])
@pytest.mark.parametrize("transposed", [False, True])
def test_layer_norm_matches_native(n, transposed):
    g = torch.Generator().manual_seed(1047)
    x = torch.randn(n, n, 128, generator=g)
    x[0, 0] = 1000.0
    x[0, 1] = 1.0 + torch.arange(128) * 1e-6
    x[0, 2] = 1000.0 + torch.arange(128) * 0.001
    x[0, 3] = 0.0
    w = torch.randn(128, generator=g)
    b = torch.randn(128, generator=g)
    stress = torch.zeros(n, n, dtype=torch.bool)
    stress[0, :4] = True
    view = x.transpose(0, 1) if transposed else x
    stress = stress.transpose(0, 1) if transposed else stress
    expected = oracle.layer_norm(view, w, b, 1e-5)
    exact = oracle.layer_norm(view.double(), w.double(), b.double(), 1e-5)
    xc = x.cuda()
    vc = xc.transpose(0, 1) if transposed else xc
    saved = xc.clone()
    with torch.inference_mode():
        actual = layer_norm.layer_norm_c128(vc, w.cuda(), b.cuda(), 1e-5)
        torch.cuda.synchronize()
    assert actual.is_contiguous() and actual.data_ptr() != xc.data_ptr()
    assert torch.equal(xc, saved)
    actual = actual.cpu()
    # ordinary rows: the fp32 native LayerNorm at the 1e-4 bar
    assert_f32_parity(f"ln n={n} transposed={transposed}", actual[~stress], expected[~stress])
    # stress rows (|mean|/std ~ 3e4, a constant row): fp32 torch itself is off by
    # ~2e-3 there, so they are held to the float64 evaluation of the formula
    torch.testing.assert_close(actual[stress].double(), exact[stress], atol=1e-5, rtol=1e-5)


def test_layer_norm_dispatch_counts_and_fallback():
    module = torch.nn.LayerNorm(128).cuda().eval()
    x = torch.randn(64, 64, 128, device="cuda")
    before = layer_norm.manifest()["counts"].get("hip-transposed", 0)
    with torch.inference_mode():
        out = layer_norm.dispatch_layer_norm(module=module, x=x.transpose(0, 1),
                                             native=lambda: pytest.fail("native"))
        torch.testing.assert_close(out, module(x.transpose(0, 1)), atol=2e-5, rtol=2e-5)
    assert layer_norm.manifest()["counts"]["hip-transposed"] == before + 1
    sentinel = object()
    module.train()
    assert layer_norm.dispatch_layer_norm(module=module, x=x, native=lambda: sentinel) is sentinel


@pytest.mark.parametrize("batch,n", [(3, 124), (16, 1000)])
def test_qkv_projection_matches_native(batch, n):
    g = torch.Generator().manual_seed(1021)
    x = torch.randn(batch, n, 128, generator=g)
    x[0, 0] = 0.0
    x[0, 1] = 100.0
    x[0, 2] = -100.0
    ws = [torch.randn(128, 128, generator=g) * 0.1 for _ in range(3)]
    p = oracle.BlockParams(None, None, ws[0], ws[1], ws[2], ws[0], None, torch.zeros(4, 128),
                           torch.zeros(128, 128), None)
    eq, ek, ev = oracle.prep_qkv(x, p, apply_scale=True)
    with torch.inference_mode():
        out = qkv_projection.qkv_projection(x.cuda(), *[w.cuda() for w in ws])
        torch.cuda.synchronize()
    views = [t.view(batch, n, 4, 32).transpose(1, 2) for t in out.unbind(0)]
    for name, actual, expected in zip("qkv", views, (eq, ek, ev)):
        assert actual.stride() == (n * 128, 32, 128, 1)
        assert_f32_parity(f"qkv {name} b={batch} n={n}", actual.cpu(), expected)


def test_sigmoid_gate_extremes_and_inputs_unchanged():
    gate = torch.linspace(-1000, 1000, 4096).reshape(32, 128)
    value = torch.randn(32, 128, generator=torch.Generator().manual_seed(3))
    gc, vc = gate.cuda(), value.cuda()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        result = attention_gate.sigmoid_mul_out(gc, vc)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    torch.testing.assert_close(result.cpu(), torch.sigmoid(gate) * value, atol=2e-6, rtol=2e-6)
    assert torch.equal(gc.cpu(), gate) and torch.equal(vc.cpu(), value)
    assert result.data_ptr() != vc.data_ptr()
    with pytest.raises(ValueError):
        attention_gate.sigmoid_mul_out(gc[:, 1:], vc[:, 1:])


@pytest.mark.parametrize("layout", ["offset8", "stride130", "rows2d"])
def test_layer_norm_other_layouts(layout):
    """Rows only 8-byte aligned (the one-wave-per-row kernel), rows whose
    stride is not a multiple of 4 floats, and a 2-D [R, 128] input with a
    ragged last row group (16 rows per group in the 16-byte-aligned kernel)."""
    g = torch.Generator().manual_seed(1063)
    n = 150
    w = torch.randn(128, generator=g)
    b = torch.randn(128, generator=g)
    if layout == "offset8":
        flat = torch.randn(n * n * 128 + 2, generator=g).cuda()
        view = flat[2:].view(n, n, 128)
        assert view.data_ptr() % 16 == 8
    elif layout == "stride130":
        view = torch.randn(n, n, 130, generator=g).cuda()[..., :128]
    else:
        view = torch.randn(n * n + 5, 128, generator=g).cuda()
    expected = oracle.layer_norm(view.cpu(), w, b, 1e-5)
    with torch.inference_mode():
        actual = layer_norm.layer_norm_c128(view, w.cuda(), b.cuda(), 1e-5)
        torch.cuda.synchronize()
    assert_f32_parity(f"ln {layout}", actual.cpu(), expected)


def test_sigmoid_gate_ragged_count():
    g = torch.Generator().manual_seed(1069)
    gate = torch.randn(37, 3, 128, generator=g) * 20
    value = torch.randn(37, 3, 128, generator=g)
    out = torch.full((37, 3, 128), float("nan")).cuda()
    from fireprot_amd import _native

    lib = _native.library()
    gc, vc = gate.cuda(), value.cuda()
    code = lib.fpx_sigmoid_mul_out(gc.data_ptr(), vc.data_ptr(), out.data_ptr(), gate.numel(),
                                   torch.cuda.current_stream().cuda_stream)
    _native.check(code, "fpx_sigmoid_mul_out")
    torch.cuda.synchronize()
    torch.testing.assert_close(out.cpu(), torch.sigmoid(gate) * value, atol=2e-6, rtol=2e-6)
