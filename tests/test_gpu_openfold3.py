"""GPU parity of the OpenFold3 consumer (fpx_attn_strided through
``fireprot_amd.openfold3``) against the oracle's native ``_attention``.

Bar (FP32): max-abs 1e-4 and rel 1e-4 elementwise against
``oracle.attention_core`` (``for b in biases: a += b`` then softmax, the order
of OpenFold3's ``_attention``), NaN positions equal.  The wire layouts are the
ones OpenFold3 hands over (adapters/openfold3/attention.py:99-119 and the
reference's layout tests tests/operators/test_openfold3_bias_layouts.py,
test_openfold3_mask_layouts.py): q/k/v as ``[B, 4, N, 32]`` views of
``[B, N, 4, 32]``, the triangle bias head-first or head-last, each as is or
transposed (ending node), the mask bias per row, broadcast, or a transposed
pair-mask view.  At B = N = 1536 the same values in every layout must give
bit-identical outputs, and sampled rows are checked against the oracle.
"""
from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import openfold3 as of3
from oracle import triangle_attention as oracle
from tests.helpers import assert_f32_parity

pytestmark = pytest.mark.gpu

BIAS_LAYOUTS = ("head_first", "head_first_t", "head_last", "head_last_t")


def bias_view(t: torch.Tensor, layout: str) -> torch.Tensor:
    """The values t[1, 4, N, N] in one of OpenFold3's memory layouts."""
    h = t[0]
    if layout == "head_first":
        return t.contiguous()
    if layout == "head_first_t":
        return h.transpose(1, 2).contiguous().transpose(1, 2).unsqueeze(0)
    if layout == "head_last":
        return h.permute(1, 2, 0).contiguous().permute(2, 0, 1).unsqueeze(0)
    if layout == "head_last_t":
        return h.permute(2, 1, 0).contiguous().permute(2, 1, 0).unsqueeze(0)
    raise ValueError(layout)


def mask_view(m: torch.Tensor, layout: str) -> torch.Tensor:
    """The values m[B|1, 1, 1, N] per row (contiguous) or as the transposed
    pair-mask view of the ending node (key stride B)."""
    if layout == "rows":
        return m.contiguous()
    if layout == "transposed":
        return m[:, 0, 0, :].t().contiguous().t()[:, None, None, :]
    raise ValueError(layout)


def qkv_view(x: torch.Tensor, layout: str) -> torch.Tensor:
    """x[B, 4, N, 32] as OpenFold3's head-last projection view, contiguous, or
    a view with channel stride 2 (served through a copy)."""
    if layout == "head_last":
        return x.transpose(1, 2).contiguous().transpose(1, 2)
    if layout == "contiguous":
        return x.contiguous()
    if layout == "channel_strided":
        wide = torch.zeros(*x.shape[:-1], 64, device=x.device, dtype=x.dtype)
        wide[..., ::2] = x
        return wide[..., ::2]
    raise ValueError(layout)


def make_case(batch, n, seed, *, mask="binary", mask_batch=None, device="cpu"):
    g = torch.Generator(device=device).manual_seed(seed)
    q = torch.randn(batch, 4, n, 32, generator=g, device=device) / 32 ** 0.5
    k = torch.randn(batch, 4, n, 32, generator=g, device=device)
    v = torch.randn(batch, 4, n, 32, generator=g, device=device)
    bias = torch.randn(1, 4, n, n, generator=g, device=device)
    rows = batch if mask_batch is None else mask_batch
    if mask == "binary":
        keep = (torch.rand(rows, 1, 1, n, generator=g, device=device) < 0.8).float()
        keep[..., 0] = 1.0
        if rows > 2:
            keep[rows // 2] = 0.0  # a fully masked row: 1e9-quantised logits
        mb = 1e9 * (keep - 1.0)
    elif mask == "moderate":  # values that are neither 0 nor -1e9
        mb = 3.0 * torch.randn(rows, 1, 1, n, generator=g, device=device)
        mb[..., ::3] = 0.0
        if rows > 1:
            mb[rows - 1] = -2.0 - torch.rand(1, 1, n, generator=g, device=device)  # no zero key
    else:
        mb = torch.zeros(rows, 1, 1, n, device=device)
    return q, k, v, mb, bias


def run(q, k, v, mb, bias, *, qkv="head_last", bias_layout="head_first", mask_layout="rows"):
    kernel = of3.StridedAttention()
    args = [qkv_view(t.cuda(), qkv) for t in (q, k, v)]
    biases = [mask_view(mb.cuda(), mask_layout), bias_view(bias.cuda(), bias_layout)]
    with torch.inference_mode():
        assert kernel.supports(*args, biases)
        out = kernel(*args, biases)
        torch.cuda.synchronize()
    assert tuple(out.shape) == tuple(q.shape)
    assert kernel.launches_submitted == 1
    return out.cpu()


def expected(q, k, v, mb, bias):
    return oracle.attention_core(q, k, v, [mb.clone(), bias.clone()])


CASES = [(1, 1, "binary"), (3, 5, "binary"), (4, 37, "binary"), (5, 124, "binary"),
         (6, 130, "binary"), (3, 257, "moderate"), (2, 1000, "binary"), (2, 1536, "binary"),
         (4, 64, "none"), (3, 200, "moderate")]


@pytest.mark.parametrize("batch,n,mask", CASES)
@pytest.mark.parametrize("bias_layout", BIAS_LAYOUTS)
def test_strided_matches_native(batch, n, mask, bias_layout):
    print(f"case of3 batch={batch} n={n} mask={mask} bias={bias_layout}", flush=True)
    q, k, v, mb, bias = make_case(batch, n, 1000 + 7 * n + batch, mask=mask)
    actual = run(q, k, v, mb, bias, bias_layout=bias_layout)
    assert_f32_parity(f"of3 b={batch} n={n} {mask} {bias_layout}", actual,
                      expected(q, k, v, mb, bias))


@pytest.mark.parametrize("qkv", ["head_last", "contiguous", "channel_strided"])
@pytest.mark.parametrize("mask_layout,mask_batch", [("rows", None), ("transposed", None),
                                                    ("rows", 1)])
def test_operand_and_mask_layouts(qkv, mask_layout, mask_batch):
    print(f"case of3 qkv={qkv} mask={mask_layout} mask_batch={mask_batch}", flush=True)
    q, k, v, mb, bias = make_case(7, 96, 77, mask_batch=mask_batch)
    actual = run(q, k, v, mb, bias, qkv=qkv, bias_layout="head_last_t", mask_layout=mask_layout)
    assert_f32_parity(f"of3 qkv={qkv} mask={mask_layout}", actual,
                      expected(q, k, v, mb.expand(7, 1, 1, 96), bias))


def test_large_logits_and_neg_inf_rows():
    """A bias scaled to logits of a few hundred, a +80 key, and a row whose
    keys are all -inf (NaN, as torch.softmax gives)."""
    q, k, v, mb, bias = make_case(4, 160, 5, mask="none")
    bias = bias * 60.0
    bias[0, 1, 3, 17] = 80.0
    mb[2, 0, 0, :] = float("-inf")
    actual = run(q, k, v, mb, bias, bias_layout="head_last")
    exp = expected(q, k, v, mb, bias)
    assert torch.isnan(actual[2]).all() and torch.isnan(exp[2]).all()
    assert_f32_parity("of3 large logits", actual, exp)


def _gpu_native(q, k, v, biases, use_high_precision=False):
    """OpenFold3's _attention arithmetic in torch on the device (the native
    function the hook captures)."""
    del use_high_precision
    a = torch.matmul(q, k.transpose(-1, -2).contiguous())
    for b in biases:
        a = a + b
    return torch.matmul(torch.softmax(a, dim=-1), v)


def test_scoped_hook_routes_eligible_calls_to_the_kernel():
    kernel = of3.StridedAttention()
    dispatcher = of3.AttentionDispatcher(kernel)
    module = SimpleNamespace(_attention=_gpu_native)
    q, k, v, mb, bias = make_case(6, 136, 9)
    args = [qkv_view(t.cuda(), "head_last") for t in (q, k, v)]
    biases = [mb.cuda(), bias_view(bias.cuda(), "head_last")]
    with of3.ScopedAttentionHook(module, dispatcher):
        with torch.inference_mode():
            fused = module._attention(*args, biases, use_high_precision=True)
            again = module._attention(*args, biases)
            # 8 heads are outside the contract: the native function runs
            wide = [torch.zeros(1, 8, 4, 32, device="cuda")] * 3
            native = module._attention(*wide, [torch.zeros(1, 1, 1, 4, device="cuda"),
                                               torch.zeros(1, 8, 4, 4, device="cuda")])
        torch.cuda.synchronize()
    assert module._attention is _gpu_native
    assert kernel.launches_submitted == 2
    assert torch.equal(fused, again)
    assert native.shape == (1, 8, 4, 32)
    assert_f32_parity("of3 hook", fused.cpu(), expected(q, k, v, mb, bias))
    selected = [d["selected"] for d in dispatcher.manifest()["registry"]["decisions"]]
    assert selected.count(of3.IMPLEMENTATION) >= 1 and "native" in selected


def test_inputs_unchanged_and_output_fresh():
    q, k, v, mb, bias = make_case(3, 72, 21)
    args = [qkv_view(t.cuda(), "head_last") for t in (q, k, v)]
    biases = [mask_view(mb.cuda(), "transposed"), bias_view(bias.cuda(), "head_first_t")]
    saved = [t.clone() for t in (*args, *biases)]
    kernel = of3.StridedAttention()
    with torch.inference_mode():
        first = kernel(*args, biases)
        second = kernel(*args, biases)
        torch.cuda.synchronize()
    assert first.data_ptr() != second.data_ptr() and torch.equal(first, second)
    for t, before in zip((*args, *biases), saved):
        assert torch.equal(t, before)
    # [B, 4, N, 32] on [B, N, 4, 32] memory: the caller's transpose is free
    assert first.transpose(1, 2).is_contiguous()


def test_c_abi_guards():
    from fireprot_amd import _native

    lib = _native.library()
    q = torch.zeros(2, 8, 4, 32, device="cuda").transpose(1, 2)
    ws = torch.empty(lib.fpx_attn_strided_workspace_bytes(2, 8), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    p = q.data_ptr()
    out = torch.empty_like(q)
    o = out.data_ptr()

    def call(n=8, batch=2, row=128, mask_sk=1, workspace=ws.data_ptr(), size=ws.numel(), ptr=p):
        return lib.fpx_attn_strided(ptr, 1024, 32, row, p, 1024, 32, row, p, 1024, 32, row,
                                    None, 0, mask_sk, None, 0, 0, 0, o, 1024, 32, row, batch, n,
                                    workspace, size, stream)

    assert call() == 0
    assert call(n=0) == 2 and call(n=4097) == 2 and call(batch=0) == 2
    assert call(row=130) == 2 and call(mask_sk=-1) == 2
    assert call(ptr=p + 4) == 3 and call(workspace=ws.data_ptr() + 64) == 3
    assert call(size=ws.numel() - 1) == 4
    assert lib.fpx_attn_strided_workspace_bytes(0, 8) == 0
    torch.cuda.synchronize()


def test_n1536_full_batch_layout_invariance_and_sampled_rows():
    """B = N = 1536 (the OpenFold3 N1536 pair stack): the ending-node wire
    layout (head-last transposed bias, transposed pair mask) and the plain
    layout of the same values give bit-identical outputs; 10 sampled rows
    match the oracle."""
    n = 1536
    print("case of3 n1536 full batch", flush=True)
    q, k, v, mb, bias = make_case(n, n, 31, device="cuda")
    kernel = of3.StridedAttention()
    with torch.inference_mode():
        plain = kernel(q.contiguous(), k.contiguous(), v.contiguous(), [mb, bias])
        ending = kernel(qkv_view(q, "head_last"), qkv_view(k, "head_last"),
                        qkv_view(v, "head_last"),
                        [mask_view(mb, "transposed"), bias_view(bias, "head_last_t")])
        torch.cuda.synchronize()
        assert torch.equal(plain, ending), "layouts of the same values disagree"
        rows = torch.tensor([0, 1, 700, n // 2, 1200, n - 1, 17, 333, 999, 1500], device="cuda")
        got = ending[rows].cpu()
        parts = [t[rows].cpu() for t in (q, k, v, mb)]
        b_cpu = bias.cpu()
    del plain, ending, q, k, v
    torch.cuda.empty_cache()
    assert torch.isfinite(got).all()  # row n // 2 is fully masked: -1e9-quantised, finite
    exp = expected(*parts, b_cpu)
    assert_f32_parity("of3 n1536 rows", got, exp)


@pytest.mark.parametrize("n,valid", [(300, 200), (640, 520)])
def test_masked_tail_skip_is_bit_identical(n, valid):
    """Keys past `valid` masked with -1e9 (at or below -2^29: their trailing
    tiles are skipped once the staged magnitudes bound the logits) or with
    -1e8 (visited, weights still exactly 0): outputs bit-identical, and both
    match the oracle."""
    print(f"case of3 skip n={n} valid={valid}", flush=True)
    q, k, v, _, bias = make_case(3, n, 41, mask="none")
    keep = (torch.arange(n) < valid).float().expand(3, 1, 1, n).contiguous()
    skipped = run(q, k, v, 1e9 * (keep - 1.0), bias)
    visited = run(q, k, v, 1e8 * (keep - 1.0), bias)
    assert torch.equal(skipped, visited)
    assert_f32_parity(f"of3 skip n={n}", skipped, expected(q, k, v, 1e9 * (keep - 1.0), bias))


def test_non_finite_masked_value_keeps_every_tile():
    """An infinite v at a masked key: the magnitude record sees it, no tile is
    skipped, and the 0 * inf of the native softmax reaches the output."""
    n, valid = 200, 100
    q, k, v, _, bias = make_case(2, n, 43, mask="none")
    v[1, 2, 150, 5] = float("inf")
    keep = (torch.arange(n) < valid).float().expand(2, 1, 1, n).contiguous()
    mb = 1e9 * (keep - 1.0)
    actual = run(q, k, v, mb, bias)
    ref = expected(q, k, v, mb, bias)
    assert torch.equal(torch.isnan(actual), torch.isnan(ref))
    assert_f32_parity("of3 inf at masked key", actual, ref)
