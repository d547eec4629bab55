"""GPU parity of triangle multiplication (fpx_tri_mul) against the oracle.

Bar (FP32): max-abs 1e-4 and rel 1e-4 elementwise against
``oracle.triangle_multiplication`` (native op order) on identical seeded
inputs; the float64 brute-force fixtures to 2e-5.  Small and medium sizes
compare every element; N = 1000, 1536 and 4096 (the largest the C ABI
accepts) compare a seeded set of rows
against the oracle's row-subset path and check full-size properties: the
incoming update equals the transposed outgoing update of z^T with the a and b
branches swapped, repeat runs are bit-identical, in-place and separate
outputs agree.  Mirrors the reference's coverage (tests/operators/
test_packed_triangle.py, test_triangle_multiplication.py): both directions,
add and overwrite aliasing, partial tiles, explicit masks, non-default
streams, constant rows and large means.
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import _native, workloads
from fireprot_amd import triangle_multiplication as htm
from fireprot_amd.registry import registry
from oracle import triangle_multiplication as tm
from tests.helpers import assert_f32_parity

pytestmark = pytest.mark.gpu


def _weights(**kw):
    return workloads.make_trimul_weights(**kw)


def _params(w):
    return tm.TriMulParams(**w)


def _hip_weights(w):
    return htm.TriMulWeights.from_tensors(**w).to("cuda")


def _mask(n, kind, seed=0):
    if kind == "none":
        return None
    if kind == "tail":
        keep = torch.arange(n) < max(1, n - max(1, n // 8))
        return (keep[:, None] & keep[None, :]).float()
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(n, n, generator=g) < 0.75).float()
    if n > 2:
        m[n // 2, :] = 0.0
        m[:, n // 3] = 0.0
    return m


def _run(z, mask, w, outgoing, **kw):
    with torch.inference_mode():
        out = htm.triangle_multiplication(z.cuda(), None if mask is None else mask.cuda(),
                                          _hip_weights(w), outgoing=outgoing, **kw)
        torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,mask", [(1, "none"), (5, "random"), (7, "tail"), (33, "random"),
                                    (64, "none"), (127, "tail"), (128, "random"),
                                    (129, "random"), (200, "tail")])
def test_small_matches_oracle(n, mask, outgoing):
    print(f"case trimul n={n} mask={mask} outgoing={outgoing}", flush=True)
    z = workloads.make_pair(n)
    m = _mask(n, mask, seed=n)
    w = _weights()
    actual = _run(z, m, w, outgoing)
    expected = tm.update(z, m, _params(w), outgoing=outgoing)
    assert_f32_parity(f"trimul n={n} {mask} out={outgoing}", actual, expected)


@pytest.mark.parametrize("outgoing", [True, False])
def test_biases_affine_and_large_means(outgoing):
    """OpenFold-style biases on all six projections, affine LayerNorms, z rows
    with |mean| >> std, and a constant row."""
    n = 96
    z = workloads.make_pair(n) * 0.01 + 1000.0
    z[3, 5, :] = 1000.0
    m = _mask(n, "random", seed=2)
    w = _weights(biases=True, affine=True)
    actual = _run(z, m, w, outgoing)
    expected = tm.update(z.double(), m.double(), _params(w).to(torch.float64),
                         outgoing=outgoing).float()
    assert torch.isfinite(actual).all()
    assert_f32_parity(f"trimul biases out={outgoing}", actual, expected)


@pytest.mark.parametrize("name", ["t5_plain", "t6_mask_affine", "t7_tail"])
def test_golden_fixtures(name):
    from tests.test_oracle_trimul import FIELDS, load_trimul_case

    z, mask, params, u_out, u_in = load_trimul_case(name, torch.float32)
    w = {k: getattr(params, k) for k in FIELDS}
    for outgoing, expected in ((True, u_out), (False, u_in)):
        actual = _run(z, mask, w, outgoing)
        torch.testing.assert_close(actual.double(), expected, atol=2e-5, rtol=1e-4)


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("add", [True, False])
def test_in_place_add_and_overwrite(outgoing, add):
    n = 150
    z = workloads.make_pair(n)
    m = _mask(n, "tail")
    w = _weights(biases=True)
    expected = tm.forward(z, m, _params(w), outgoing=outgoing, add=add)
    zc = z.cuda()
    ptr = zc.data_ptr()
    with torch.inference_mode():
        out = htm.triangle_multiplication(zc, m.cuda(), _hip_weights(w), outgoing=outgoing,
                                          out=zc, accumulate=add)
        torch.cuda.synchronize()
    assert out.data_ptr() == ptr
    assert_f32_parity(f"in place add={add} out={outgoing}", zc.cpu(), expected)


def test_strided_input_output_and_alias_guard():
    n = 70
    base = workloads.make_pair(n + 3)
    z = base[1:n + 1, 2:n + 2]          # row stride (n + 3) * 128, not contiguous
    w = _weights()
    expected = tm.update(z, None, _params(w), outgoing=False)
    storage = torch.full((n * n * 128 * 2 + 8192,), 7.5, device="cuda")
    out = storage[4096:4096 + 2 * n * n * 128].view(n, 2 * n, 128)[:, ::2]
    zc = base.cuda()[1:n + 1, 2:n + 2]
    saved = zc.clone()
    with torch.inference_mode():
        htm.triangle_multiplication(zc, None, _hip_weights(w), outgoing=False, out=out)
        torch.cuda.synchronize()
    assert torch.equal(zc, saved)
    assert bool((storage[:4096] == 7.5).all()) and bool((storage[-4096:] == 7.5).all())
    assert bool((storage[4096:4096 + 2 * n * n * 128].view(n, 2 * n, 128)[:, 1::2] == 7.5).all())
    assert_f32_parity("strided", out.cpu(), expected)
    # out == z with different strides is refused before any launch
    lib = _native.library()
    wt = _hip_weights(w)
    zz = torch.zeros(n, n, 128, device="cuda")
    ws = torch.empty(htm.workspace_bytes(n), dtype=torch.uint8, device="cuda")
    code = lib.fpx_tri_mul(zz.data_ptr(), n * 128, 128, None, 0, 0, None, None, 1e-5,
                           wt.w_abpg.data_ptr(), None, None, None, 1e-5, wt.w_z.data_ptr(), None,
                           wt.w_g.data_ptr(), None, n, 128, 128, 1, 0, zz.data_ptr(), 128,
                           n * 128, ws.data_ptr(), ws.numel(),
                           torch.cuda.current_stream().cuda_stream)
    assert code == 2


def test_nondefault_stream_and_queued_calls():
    n = 100
    z, m, w = workloads.make_pair(n), _mask(n, "random", 4), _weights()
    expected = tm.update(z, m, _params(w), outgoing=True)
    zc, mc, wt = z.cuda(), m.cuda(), _hip_weights(w)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.inference_mode(), torch.cuda.stream(stream):
        outs = [htm.triangle_multiplication(zc, mc, wt, outgoing=True) for _ in range(3)]
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for out in outs:
        assert_f32_parity("queued", out.cpu(), expected)


def _swap(w):
    s = dict(w)
    for x in ("w_{}_p", "w_{}_g", "b_{}_p", "b_{}_g"):
        s[x.format("a")], s[x.format("b")] = w[x.format("b")], w[x.format("a")]
    return s


@pytest.mark.parametrize("n", [1000, 1536])
def test_long_rows_and_direction_identity(n):
    print(f"case trimul long n={n}", flush=True)
    z = workloads.make_pair(n)
    m = _mask(n, "tail")
    w = _weights()
    zc, mc, wt = z.cuda(), m.cuda(), _hip_weights(w)
    g = torch.Generator().manual_seed(n)
    rows = torch.unique(torch.cat([torch.tensor([0, 1, n // 2, n - 1, n - n // 8]),
                                   torch.randint(0, n, (6,), generator=g)]))
    with torch.inference_mode():
        out = htm.triangle_multiplication(zc, mc, wt, outgoing=True)
        inc = htm.triangle_multiplication(zc, mc, wt, outgoing=False)
        again = htm.triangle_multiplication(zc, mc, wt, outgoing=False)
        mirror = htm.triangle_multiplication(zc.transpose(0, 1).contiguous(),
                                             mc.t().contiguous(), _hip_weights(_swap(w)),
                                             outgoing=True).transpose(0, 1)
        torch.cuda.synchronize()
        assert torch.equal(inc, again), "not deterministic"
        assert torch.isfinite(out).all() and torch.isfinite(inc).all()
        torch.testing.assert_close(inc, mirror, atol=1e-5, rtol=1e-5)
        got_out, got_in = out[rows.cuda()].cpu(), inc[rows.cuda()].cpu()
    del out, inc, again, mirror
    torch.cuda.empty_cache()
    p = _params(w)
    assert_f32_parity(f"n={n} outgoing rows", got_out, tm.update(z, m, p, outgoing=True,
                                                                 rows=rows))
    assert_f32_parity(f"n={n} incoming rows", got_in, tm.update(z, m, p, outgoing=False,
                                                                rows=rows))


@pytest.mark.timeout(600)
def test_maximum_n4096_rows():
    """N = 4096, the largest size the C ABI accepts (a and b of 2^31 values
    each): both directions on five rows against the oracle's row-subset path,
    and a repeat run bit-identical.  z is drawn on the GPU (a seeded device
    generator) and copied to the host for the oracle."""
    n = 4096
    print(f"case trimul maximum n={n}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(419 + n)
    zc = torch.randn(n, n, 128, generator=g, device="cuda")
    m = _mask(n, "tail")
    mc = m.cuda()
    w = _weights()
    wt = _hip_weights(w)
    valid = int(m[0].sum())
    gr = torch.Generator().manual_seed(n)
    rows = torch.tensor(sorted({0, valid - 1, valid, n - 1,
                                int(torch.randint(0, valid, (1,), generator=gr))}))
    got = {}
    with torch.inference_mode():
        for outgoing in (True, False):
            out = htm.triangle_multiplication(zc, mc, wt, outgoing=outgoing)
            assert torch.isfinite(out).all()
            got[outgoing] = out[rows.cuda()].cpu()
            if not outgoing:
                again = htm.triangle_multiplication(zc, mc, wt, outgoing=False)
                torch.cuda.synchronize()
                assert torch.equal(out, again), "not deterministic"
                del again
            del out
    z = zc.cpu()
    del zc
    torch.cuda.empty_cache()
    p = _params(w)
    for outgoing in (True, False):
        assert_f32_parity(f"n={n} outgoing={outgoing} rows", got[outgoing],
                          tm.update(z, m, p, outgoing=outgoing, rows=rows))


class _Module(torch.nn.Module):
    """The attribute surface of Protenix's TriangleMultiplicativeUpdate."""

    def __init__(self, w, outgoing):
        super().__init__()
        self.c_z = self.c_hidden = 128
        self._outgoing = outgoing
        self.layer_norm_in = torch.nn.LayerNorm(128)
        self.layer_norm_out = torch.nn.LayerNorm(128)
        for name in ("a_p", "a_g", "b_p", "b_g", "z", "g"):
            layer = torch.nn.Linear(128, 128, bias=False)
            layer.weight.data.copy_(w[f"w_{name}"])
            setattr(self, f"linear_{name}", layer)


def test_dispatch_through_registry_in_place_and_native_fallback():
    n = 90
    z, m, w = workloads.make_pair(n), _mask(n, "random", 6), _weights()
    module = _Module(w, outgoing=False).cuda().eval()
    expected = tm.forward(z, m, _params(w), outgoing=False, add=True)
    zc = z.cuda()
    registry.clear_runtime_state()
    calls = []
    with torch.inference_mode():
        result = htm.dispatch_triangle_multiplication(
            module=module, z=zc, mask=m.cuda(), inplace_safe=True, add_with_inplace=True,
            inplace_chunk_size=256, native=lambda **_: calls.append(1))
        torch.cuda.synchronize()
    assert result.data_ptr() == zc.data_ptr() and not calls
    assert_f32_parity("dispatch", zc.cpu(), expected)
    assert registry.count(htm.OPERATION, htm.IMPLEMENTATION) == 1
    # autograd enabled: the native function runs
    result = htm.dispatch_triangle_multiplication(
        module=module, z=zc, mask=None, inplace_safe=True, add_with_inplace=True,
        inplace_chunk_size=256, native=lambda **_: "native")
    assert result == "native"
    # not in place: a fresh update tensor, z untouched
    before = zc.clone()
    with torch.inference_mode():
        update = htm.dispatch_triangle_multiplication(
            module=module, z=zc, mask=m.cuda(), inplace_safe=False, add_with_inplace=False,
            inplace_chunk_size=None, native=lambda **_: None)
        torch.cuda.synchronize()
    assert torch.equal(zc, before) and update.data_ptr() != zc.data_ptr()
    assert_f32_parity("dispatch update", update.cpu(),
                      tm.update(before.cpu(), m, _params(w), outgoing=False))
