"""GPU parity of the pair transition (fpx_transition) against the oracle.

Bar (FP32): elementwise max-abs 1e-4 and rel 1e-4 against
``oracle.transition`` (native op order) on identical seeded inputs; the
float64 brute-force fixtures to 1e-6 of their largest value.  Covers partial
row tiles, strided 3-D and flat inputs, the in-place residual form, the
N = 1536 pair stack (sampled rows against the oracle, repeat runs
bit-identical), the N = 4096 stack in place, registry dispatch and the native fallback (the reference's
tests/backends/test_recycle.py and tests/operators/test_long1536_epilogues.py
cover the same surface).
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import workloads
from fireprot_amd import transition as htr
from fireprot_amd.registry import registry
from oracle import transition as tr
from tests.helpers import assert_f32_parity

pytestmark = pytest.mark.gpu


def _params(w):
    return tr.TransitionParams(**w)


def _hip(w):
    return htr.TransitionWeights.from_tensors(**w).to("cuda")


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (7, 33), (40, 40), (64, 64), (130, 131)])
def test_matches_oracle(shape):
    print(f"case transition shape={shape}", flush=True)
    g = torch.Generator().manual_seed(shape[0] * 1000 + shape[1])
    z = torch.randn(*shape, 128, generator=g)
    w = workloads.make_transition_weights(affine=True)
    with torch.inference_mode():
        actual = htr.transition(z.cuda(), _hip(w))
        torch.cuda.synchronize()
    assert_f32_parity(f"transition {shape}", actual.cpu(), tr.transition(z, _params(w)))


@pytest.mark.parametrize("name", ["tr3_plain", "tr4_affine"])
def test_golden_fixtures(name):
    from tests.test_oracle_transition import FIELDS, load_transition_case

    z, p, expected = load_transition_case(name, torch.float32)
    w = {k: getattr(p, k) for k in FIELDS}
    with torch.inference_mode():
        actual = htr.transition(z.cuda(), _hip(w)).cpu()
    torch.testing.assert_close(actual.double(), expected,
                               atol=1e-6 * float(expected.abs().max()), rtol=1e-4)


def test_strided_flat_and_in_place():
    w = workloads.make_transition_weights()
    base = workloads.make_pair(70)
    z = base[2:62, 5:65]                      # strided rows
    expected = tr.transition(z, _params(w))
    zc = base.cuda()[2:62, 5:65]
    wt = _hip(w)
    with torch.inference_mode():
        strided = htr.transition(zc, wt)
        flat = htr.transition(zc.reshape(-1, 128), wt)      # contiguous copy, [rows, 128]
        batched = htr.transition(zc.unsqueeze(0).contiguous(), wt)   # [1, I, J, 128]
        target = zc.clone()
        ptr = target.data_ptr()
        htr.pair_transition_residual(target, wt)
        torch.cuda.synchronize()
    assert_f32_parity("strided", strided.cpu(), expected)
    assert_f32_parity("flat", flat.cpu().view(60, 60, 128), expected)
    assert_f32_parity("batched", batched.cpu()[0], expected)
    assert target.data_ptr() == ptr
    assert_f32_parity("in place", target.cpu(), z + expected)


def test_x_offset_by_two_floats():
    """x rows are read as 16-byte vectors: an x that starts 8 bytes past a
    16-byte boundary is refused by the C ABI (status 3, before any launch)
    and copied to an aligned buffer by the host wrapper, with the same
    result; an odd-multiple-of-2 row stride is refused with status 2."""
    from fireprot_amd import _native

    n = 24
    w = workloads.make_transition_weights(affine=True)
    z = workloads.make_pair(n)
    expected = tr.transition(z, _params(w))
    wt = _hip(w)
    buf = torch.zeros(n * n * 128 + 8, device="cuda")
    x = buf[2:2 + n * n * 128].view(n, n, 128)
    x.copy_(z.cuda())
    assert x.data_ptr() % 16 == 8
    lib = _native.library()
    size = lib.fpx_transition_workspace_bytes(n, n, 128, 4)
    ws = torch.empty(size, dtype=torch.uint8, device="cuda")
    out = torch.empty(n, n, 128, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream

    def call(ptr, si, sj):
        return lib.fpx_transition(ptr, n, n, si, sj, wt.ln_w.data_ptr(), wt.ln_b.data_ptr(),
                                  wt.eps, wt.w_a.data_ptr(), wt.w_b.data_ptr(),
                                  wt.w_o.data_ptr(), 128, 4, 0, out.data_ptr(), n * 128, 128,
                                  ws.data_ptr(), ws.numel(), stream)

    assert call(x.data_ptr(), n * 128, 128) == 3
    assert call(buf.data_ptr(), n * 128 + 2, 128) == 2
    with torch.inference_mode():
        actual = htr.transition(x, wt)
        torch.cuda.synchronize()
    assert_f32_parity("x offset by 2 floats", actual.cpu(), expected)


def test_n1536_rows_and_determinism():
    n = 1536
    print("case transition n1536", flush=True)
    z = workloads.make_pair(n)
    w = workloads.make_transition_weights()
    zc = z.cuda()
    wt = _hip(w)
    with torch.inference_mode():
        first = htr.transition(zc, wt)
        second = htr.transition(zc, wt)
        torch.cuda.synchronize()
        assert torch.equal(first, second)
        assert torch.isfinite(first).all()
        rows = torch.tensor([0, 1, 700, 1535])
        got = first[rows.cuda()].cpu()
    del first, second
    assert_f32_parity("n1536 rows", got, tr.transition(z[rows], _params(w)))


@pytest.mark.timeout(600)
def test_maximum_n4096_rows_in_place():
    """N = 4096, the largest pair size (16.8 M rows, a 34 GB hidden layer in
    the workspace): the in-place residual update on five pair rows against
    the oracle.  z is drawn on the GPU (a seeded device generator)."""
    n = 4096
    print(f"case transition maximum n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(419 + n)
    zc = torch.randn(n, n, 128, generator=g, device="cuda")
    rows = torch.tensor([0, 1, 2047, 3000, n - 1])
    z_rows = zc[rows.cuda()].cpu()
    w = workloads.make_transition_weights()
    with torch.inference_mode():
        out = htr.transition(zc, _hip(w), out=zc, accumulate=True)
        torch.cuda.synchronize()
        assert out.data_ptr() == zc.data_ptr()
        assert torch.isfinite(zc).all()
        got = zc[rows.cuda()].cpu()
    del zc, out
    torch.cuda.empty_cache()
    assert_f32_parity(f"n={n} rows in place", got, z_rows + tr.transition(z_rows, _params(w)))


def _module(w):
    norm = torch.nn.LayerNorm(128)
    norm.weight.data.copy_(w["ln_w"])
    norm.bias.data.copy_(w["ln_b"])
    layers = {}
    for name, key, shape in (("linear_no_bias_a", "w_a", (128, 512)),
                             ("linear_no_bias_b", "w_b", (128, 512)),
                             ("linear_no_bias", "w_o", (512, 128))):
        layer = torch.nn.Linear(*shape, bias=False)
        layer.weight.data.copy_(w[key])
        layers[name] = layer.cuda()
    return SimpleNamespace(training=False, n=4, c_in=128, layernorm1=norm.cuda(), **layers)


def test_dispatch_and_native_fallback():
    w = workloads.make_transition_weights(affine=True)
    module = _module(w)
    z = workloads.make_pair(50)
    registry.clear_runtime_state()
    with torch.inference_mode():
        out = htr.dispatch_transition(module=module, x=z.cuda(), native=lambda **_: "native")
        torch.cuda.synchronize()
    assert_f32_parity("dispatch", out.cpu(), tr.transition(z, _params(w)))
    assert registry.count(htr.OPERATION, htr.IMPLEMENTATION) == 1
    # autograd on, or a module of another width: the native function runs
    assert htr.dispatch_transition(module=module, x=z.cuda(), native=lambda **_: "native") == "native"
    other = SimpleNamespace(**{**vars(module), "n": 2})
    with torch.inference_mode():
        assert htr.dispatch_transition(module=other, x=z.cuda(),
                                       native=lambda **_: "native") == "native"
