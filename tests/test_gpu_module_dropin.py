"""The module-level drop-in on the GPU, through the installers.

Protenix-shaped and AtlasFold-shaped ``nn.Module`` classes (the attribute
layouts ``BlockWeights.from_protenix`` / ``from_atlasfold`` read:
patches/protenix/0005-*.patch:32-45, adapters/atlasfold/runtime.py:38-70) are
built on the GPU with the seeded weights of the workloads, hooked with
``hooks.install_protenix`` / ``hooks.AtlasFoldHooks``, and called as the
models call them: ``module(z, mask)`` returning dz.  Their own forwards fail
the test if they run, so every call must take the HIP block candidate; the
registry's selection counts confirm it.  Results are held to the FP32 bar of
tests/test_gpu_fp32_accuracy.py against the float64 oracle: C2 (N=512, last
51 residues masked) in full for both nodes through the Protenix layout, C4
(N=1536, 184-residue tail, bias x8) on sampled rows for both nodes through
the AtlasFold layout (batched ``[1, N, N, 128]`` z with a boolean mask).  The
route's workspace comes from the per-device cache: one buffer, reused by
every call.
"""
from __future__ import annotations

import pytest
import torch

from fireprot_amd import hooks, workloads
from fireprot_amd import triangle_attention as ta
from fireprot_amd import workspace as ws_cache
from fireprot_amd.registry import registry
from tests.test_gpu_block import _sample_rows
from tests.test_gpu_fp32_accuracy import _check_regions

pytestmark = pytest.mark.gpu


def _linear(w, bias=None):
    layer = torch.nn.Linear(w.shape[1], w.shape[0], bias=bias is not None)
    with torch.no_grad():
        layer.weight.copy_(w)
        if bias is not None:
            layer.bias.copy_(bias)
    return layer


def _layer_norm(w):
    ln = torch.nn.LayerNorm(128)
    with torch.no_grad():
        ln.weight.copy_(w["ln_w"])
        ln.bias.copy_(w["ln_b"])
    return ln


class _Mha(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.linear_q, self.linear_k = _linear(w["w_q"]), _linear(w["w_k"])
        self.linear_v, self.linear_g = _linear(w["w_v"]), _linear(w["w_g"], w["b_g"])
        self.linear_o = _linear(w["w_o"], w["b_o"])
        self.no_heads, self.c_hidden = 4, 32


class ProtenixTriangleAttention(torch.nn.Module):
    def __init__(self, w, starting):
        super().__init__()
        self.starting = starting
        self.layer_norm = _layer_norm(w)
        self.linear = _linear(w["w_bias"])
        self.mha = _Mha(w)
        self.inf = 1e9

    def forward(self, x, mask=None, chunk_size=None):
        pytest.fail("the native TriangleAttention.forward ran")


class AtlasFoldStart(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.layernorm = _layer_norm(w)
        self.linear_qkv = _linear(torch.cat([w["w_q"], w["w_k"], w["w_v"]], 0))
        self.linear_bias = _linear(w["w_bias"])
        self.linear_g = _linear(w["w_g"])
        self.linear_out = _linear(w["w_o"])
        self.num_heads, self.channel_hidden, self.inf = 4, 32, 1e9
        self.scale = 32 ** -0.5

    def forward(self, z, mask, kernel_backend="torch"):
        pytest.fail("the native AtlasFold triangle forward ran")


class AtlasFoldEnd(AtlasFoldStart):
    pass


class _AtlasFoldModel(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.tri_attn_start = AtlasFoldStart(w)
        self.tri_attn_end = AtlasFoldEnd(w)


@pytest.fixture
def protenix_cls():
    cls = type("TriangleAttention", (ProtenixTriangleAttention,),
               {"forward": ProtenixTriangleAttention.forward})
    hooks.install_protenix(cls)
    yield cls
    hooks.uninstall_protenix()


def test_protenix_layout_c2_full_both_nodes(protenix_cls):
    cfg = workloads.CONFIGS["c2"]
    z, mask, w = workloads.make_inputs(cfg)
    zc, mc = z.cuda(), mask.cuda()
    registry.clear_runtime_state()
    ws_cache.release()
    rows = torch.arange(cfg.n)
    for ending in (False, True):
        print(f"case protenix {cfg.name} ending={ending}", flush=True)
        module = protenix_cls(w, starting=not ending).cuda().eval()
        with torch.inference_mode():
            dz = module(zc, mc)
            torch.cuda.synchronize()
        x_frame = (dz.transpose(0, 1) if ending else dz).cpu()
        _check_regions(f"protenix {cfg.name} ending={ending}", x_frame, z, mask, w, ending, rows,
                       cfg.valid)
    assert registry.count(ta.BLOCK_OPERATION, ta.BLOCK_IMPLEMENTATION) == 2
    assert len(ws_cache.manifest()) == 1


def test_atlasfold_layout_c4_rows_both_nodes():
    cfg = workloads.CONFIGS["c4"]
    z, mask, w = workloads.make_inputs(cfg)
    model = _AtlasFoldModel(w).cuda().eval()
    h = hooks.AtlasFoldHooks(model, starting_cls=AtlasFoldStart, ending_cls=AtlasFoldEnd)
    zc = z.cuda()[None]
    mc = mask.cuda().bool()[None]
    rows = _sample_rows(cfg.n, cfg.valid)
    registry.clear_runtime_state()
    ws_cache.release()
    try:
        for ending, module in ((False, model.tri_attn_start), (True, model.tri_attn_end)):
            print(f"case atlasfold {cfg.name} ending={ending} rows={rows.tolist()}", flush=True)
            with torch.inference_mode():
                dz = module(zc, mc)
                assert dz.shape == zc.shape
                x_frame = dz[0].transpose(0, 1) if ending else dz[0]
                picked = x_frame[rows.cuda()].cpu()
                torch.cuda.synchronize()
            del dz, x_frame
            buffers = ws_cache.manifest()
            assert len(buffers) == 1 and list(buffers.values())[0] >= ta.workspace_bytes(cfg.n)
            _check_regions(f"atlasfold {cfg.name} ending={ending}", picked, z, mask, w, ending,
                           rows, cfg.valid)
    finally:
        h.uninstall()
        ws_cache.release()
        torch.cuda.empty_cache()
    assert h.counts == {"dispatched": 2, "kept": 0}
    assert registry.count(ta.BLOCK_OPERATION, ta.BLOCK_IMPLEMENTATION) == 2


def test_cached_workspace_is_reused_across_calls(protenix_cls):
    n = 160
    z = workloads.make_pair(n).cuda()
    w = workloads.make_weights()
    module = protenix_cls(w, starting=True).cuda().eval()
    ws_cache.release()
    with torch.inference_mode():
        first = module(z)
        buf = ws_cache.get(z.device, 1, purpose="block")
        second = module(z)
        torch.cuda.synchronize()
    assert ws_cache.get(z.device, 1, purpose="block").data_ptr() == buf.data_ptr()
    assert torch.equal(first, second)
    ws_cache.release()


def test_protenix_layout_bf16_module_both_nodes(protenix_cls):
    """A bfloat16 model (module weights, z and mask in bfloat16) through the
    installed hook takes the BF16 block candidate; both nodes at N = 160 with
    a 20-residue padding tail stay within 2e-2 (of the largest value) of the
    native path run on bfloat16 tensors, the BF16 bar of
    tests/test_gpu_bf16.py."""
    from oracle import triangle_attention as oracle

    n, valid = 160, 140
    z = workloads.make_pair(n)
    mask = workloads.make_mask(n, valid)
    w = workloads.make_weights()
    zc = z.to(torch.bfloat16).cuda()
    mc = mask.to(torch.bfloat16).cuda()
    registry.clear_runtime_state()
    ws_cache.release()
    for ending in (False, True):
        print(f"case protenix bf16 n={n} ending={ending}", flush=True)
        module = protenix_cls(w, starting=not ending).cuda().eval().to(torch.bfloat16)
        with torch.inference_mode():
            dz = module(zc, mc)
            torch.cuda.synchronize()
        assert dz.dtype == torch.bfloat16
        native = oracle.block_bf16(z, mask, oracle.BlockParams(**w), ending=ending)
        rel = ((dz.float().cpu() - native.float()).abs().max() / native.float().abs().max()).item()
        print(f"protenix bf16 ending={ending}: rel vs native-bf16 {rel:.2e}", flush=True)
        assert rel <= 2e-2
    assert registry.count(ta.BLOCK_OPERATION, ta.BLOCK_BF16_IMPLEMENTATION) == 2
    assert registry.count(ta.BLOCK_OPERATION, ta.BLOCK_IMPLEMENTATION) == 0
    ws_cache.release()
