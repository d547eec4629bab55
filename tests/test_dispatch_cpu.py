"""Capability predicates and native fallback of the dispatch surfaces on the
CPU (mirrors tests/operators/test_triangle_attention.py:99-189,
test_ck_attention.py:14-41 and the hook fallback tests of the reference)."""
from __future__ import annotations

import dataclasses
from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import _native, attention_gate, block, layer_norm, pair_layout, qkv_projection
from fireprot_amd import triangle_attention as ta
from fireprot_amd.registry import OperationSignature, registry


def _core_signature(**change):
    n = 1536
    base = dict(operation=ta.OPERATION, device_type="cuda", architecture="gfx950",
                dtype="float32", shape=(512, 4, n, 32), layout="strided", mode="inference",
                mask="triangle-bias", inplace=False,
                attributes={"bias_shapes": repr(((1, 4, n, n),)),
                            "qkv_strides": repr(((n * 128, 32, 128, 1),) * 3),
                            "ck_tile_compatible": True})
    base.update(change)
    return OperationSignature.create(**base)


def test_core_capability_accepts_validated_signature(monkeypatch):
    monkeypatch.setattr(_native, "available", lambda: True)
    assert ta._supports_core(_core_signature()) is True
    masked = _core_signature(mask="additive-mask-and-triangle-bias", attributes={
        "bias_shapes": repr(((512, 1, 1, 1536), (1, 4, 1536, 1536))),
        "qkv_strides": repr(((1536 * 128, 32, 128, 1),) * 3), "ck_tile_compatible": True})
    assert ta._supports_core(masked) is True
    for change in (dict(device_type="cpu"), dict(architecture="gfx90a"),
                   dict(dtype="bfloat16"), dict(mode="training"), dict(shape=(512, 8, 1536, 16)),
                   dict(shape=(512, 4, 1534, 32))):
        assert ta._supports_core(_core_signature(**change))[0] is False
    sig = _core_signature()
    for key, value in (("ck_tile_compatible", "False"), ("qkv_strides", "other"),
                       ("bias_shapes", repr(((1, 4, 7, 7),)))):
        attributes = dict(sig.attributes)
        attributes[key] = value
        changed = dataclasses.replace(sig, attributes=tuple(sorted(attributes.items())))
        assert ta._supports_core(changed)[0] is False
    monkeypatch.setattr(_native, "available", lambda: False)
    assert ta._supports_core(sig) == (False, "HIP extension unavailable")


def test_core_dispatch_falls_back_for_cpu_tensors():
    q = torch.randn(5, 4, 8, 32).transpose(1, 2).contiguous().transpose(1, 2)
    biases = [torch.zeros(5, 1, 1, 8), torch.zeros(1, 4, 8, 8)]
    registry.clear_runtime_state()
    with torch.inference_mode():
        result = ta.dispatch_triangle_attention(module=SimpleNamespace(training=False), q=q, k=q,
                                                v=q, biases=biases, native=lambda **_: "native")
    assert result == "native"
    decision = registry.manifest()["decisions"][0]
    assert decision["signature"]["mode"] == "inference"
    assert decision["rejected"][0]["reason"] == "device is not CUDA/HIP"
    with torch.enable_grad():
        qg = q.clone().requires_grad_()
        ta.dispatch_triangle_attention(module=SimpleNamespace(training=False), q=qg, k=q, v=q,
                                       biases=biases, native=lambda **_: None)
    modes = {d["signature"]["mode"] for d in registry.manifest()["decisions"]}
    assert modes == {"inference", "training"}


class _Linear(torch.nn.Linear):
    pass


def _protenix_like(bias_g=True):
    mha = SimpleNamespace(linear_q=torch.nn.Linear(128, 128, bias=False),
                          linear_k=torch.nn.Linear(128, 128, bias=False),
                          linear_v=torch.nn.Linear(128, 128, bias=False),
                          linear_g=torch.nn.Linear(128, 128, bias=bias_g),
                          linear_o=torch.nn.Linear(128, 128), no_heads=4, c_hidden=32)
    return SimpleNamespace(layer_norm=torch.nn.LayerNorm(128), linear=torch.nn.Linear(128, 4, bias=False),
                           mha=mha, inf=1e9, training=False)


def test_block_weights_from_protenix_and_atlasfold():
    m = _protenix_like()
    w = block.BlockWeights.from_protenix(m)
    assert w.w_qkvg.shape == (512, 128) and w.w_qkvg.is_contiguous()
    assert torch.equal(w.w_qkvg[256:384], m.mha.linear_v.weight)
    assert torch.equal(w.b_g, m.mha.linear_g.bias) and w.inf == 1e9 and w.eps == 1e-5
    m.mha.linear_q = torch.nn.Linear(128, 128)
    with pytest.raises(ValueError):
        block.BlockWeights.from_protenix(m)
    a = SimpleNamespace(layernorm=torch.nn.LayerNorm(128), linear_qkv=torch.nn.Linear(128, 384, bias=False),
                        linear_bias=torch.nn.Linear(128, 4, bias=False),
                        linear_g=torch.nn.Linear(128, 128, bias=False),
                        linear_out=torch.nn.Linear(128, 128, bias=False), inf=1e9)
    w = block.BlockWeights.from_atlasfold(a)
    assert torch.equal(w.w_qkvg[:384], a.linear_qkv.weight) and w.b_g is None and w.b_o is None


def test_block_dispatch_falls_back_on_cpu_and_reports_reason():
    m = _protenix_like()
    z = torch.randn(8, 8, 128)
    registry.clear_runtime_state()
    with torch.inference_mode():
        assert ta.dispatch_triangle_attention_block(module=m, z=z, mask=None, ending=False,
                                                    native=lambda **_: "native") == "native"
    decision = registry.manifest()["decisions"][0]
    assert decision["selected"] == "native"
    assert decision["rejected"][0]["reason"] == "device is not CUDA/HIP"
    assert ta.block_eligible(m, z, None) == (False, "z is not a float32 or bfloat16 HIP tensor")


def test_block_dispatch_calls_a_preferred_candidate_with_the_hook_arguments():
    """A candidate registered above the HIP block gets the call with the
    reference hook's keyword arguments (the packed-weights shortcut applies
    only when the registry selects this package's block)."""
    m = _protenix_like()
    z = torch.randn(8, 8, 128)
    seen = {}

    def override(**kwargs):
        seen.update(kwargs)
        return "override"

    registry.register(operation=ta.BLOCK_OPERATION, name="user-override", function=override,
                      supports=lambda signature: True, priority=99, version="1")
    try:
        registry.clear_runtime_state()
        with torch.inference_mode():
            native = lambda **_: "native"  # noqa: E731
            assert ta.dispatch_triangle_attention_block(module=m, z=z, mask=None, ending=True,
                                                        native=native) == "override"
        assert set(seen) == {"module", "z", "mask", "ending", "native"}
        assert seen["module"] is m and seen["z"] is z and seen["ending"] is True
        assert seen["native"] is native
        assert registry.count(ta.BLOCK_OPERATION, "user-override") == 1
    finally:
        registry.unregister(ta.BLOCK_OPERATION, "user-override")
        registry.clear_runtime_state()


def test_block_entry_raises_without_a_device():
    z = torch.randn(4, 4, 128)
    w = block.BlockWeights.from_protenix(_protenix_like())
    with pytest.raises((ValueError, RuntimeError)):
        block.triangle_attention_block(z, None, w)


def test_stage_hooks_fall_back_on_cpu():
    sentinel = object()
    module = torch.nn.LayerNorm(128).eval()
    x = torch.randn(4, 4, 128)
    with torch.inference_mode():
        assert layer_norm.dispatch_layer_norm(module=module, x=x, native=lambda: sentinel) is sentinel
    attn = SimpleNamespace(training=False, no_heads=4, c_hidden=32)
    assert qkv_projection.prepare(module=attn, q_x=x, kv_x=x, apply_scale=True,
                                  native=lambda: sentinel) is sentinel
    assert attention_gate.wrap_up(module=SimpleNamespace(training=False, linear_g=None), o=None,
                                  x=x, native=lambda: sentinel) is sentinel
    y = pair_layout.transpose_pair(x, training=False)
    assert y.is_contiguous() and y.data_ptr() != x.data_ptr()
    assert torch.equal(y, x.transpose(0, 1))


def test_registered_implementations():
    impl = registry.manifest()["implementations"]
    assert impl[ta.OPERATION][0]["name"] == ta.IMPLEMENTATION
    assert {c["name"] for c in impl[ta.BLOCK_OPERATION]} == {ta.BLOCK_IMPLEMENTATION,
                                                             ta.BLOCK_BF16_IMPLEMENTATION}


def _trimul_signature(**change):
    from fireprot_amd import triangle_multiplication as htm

    base = dict(operation=htm.OPERATION, device_type="cuda", architecture="gfx950",
                dtype="float32", shape=(1536, 1536, 128), layout="contiguous",
                mode="inference", mask="dense", inplace=True,
                attributes={"c_z": 128, "c_hidden": 128, "eligible": True, "reason": "",
                            "direction": "incoming", "add_with_inplace": True})
    base.update(change)
    return OperationSignature.create(**base)


def test_trimul_capability(monkeypatch):
    from fireprot_amd import triangle_multiplication as htm

    monkeypatch.setattr(_native, "available", lambda: True)
    assert htm._supports(_trimul_signature()) is True
    for change in (dict(device_type="cpu"), dict(architecture="gfx90a"), dict(dtype="bfloat16"),
                   dict(mode="training"),
                   dict(attributes={"c_z": 128, "c_hidden": 64, "eligible": True}),
                   dict(attributes={"c_z": 128, "c_hidden": 128, "eligible": False,
                                    "reason": "z rows are not 16-byte aligned"})):
        assert htm._supports(_trimul_signature(**change))[0] is False
    monkeypatch.setattr(_native, "available", lambda: False)
    assert htm._supports(_trimul_signature()) == (False, "HIP extension unavailable")


def test_trimul_dispatch_falls_back_for_cpu_tensors():
    from fireprot_amd import triangle_multiplication as htm

    module = SimpleNamespace(training=False, c_z=128, c_hidden=128, _outgoing=True)
    registry.clear_runtime_state()
    with torch.no_grad():
        result = htm.dispatch_triangle_multiplication(
            module=module, z=torch.zeros(4, 4, 128), mask=None, inplace_safe=True,
            add_with_inplace=True, inplace_chunk_size=256, native=lambda **_: "native")
    assert result == "native"
    decision = registry.manifest()["decisions"][0]
    assert decision["selected"] == "native"
    assert decision["signature"]["attributes"]["direction"] == "outgoing"
    ok, reason = htm.eligible(module, torch.zeros(4, 4, 128), None)
    assert not ok and "HIP" in reason


def test_transition_capability_and_cpu_fallback(monkeypatch):
    from fireprot_amd import transition as htr

    monkeypatch.setattr(_native, "available", lambda: True)
    base = dict(operation=htr.OPERATION, device_type="cuda", architecture="gfx950",
                dtype="float32", shape=(1536, 1536, 128), layout="contiguous", mode="inference",
                mask="none", inplace=False,
                attributes={"expansion": 4, "c_in": 128, "eligible": True, "reason": ""})
    assert htr._supports(OperationSignature.create(**base)) is True
    for change in (dict(device_type="cpu"), dict(architecture="gfx942"), dict(dtype="float64"),
                   dict(mode="training"),
                   dict(attributes={"expansion": 2, "c_in": 128, "eligible": True})):
        assert htr._supports(OperationSignature.create(**(base | change)))[0] is False
    module = SimpleNamespace(training=False, n=4, c_in=128)
    registry.clear_runtime_state()
    with torch.inference_mode():
        assert htr.dispatch_transition(module=module, x=torch.randn(5, 5, 128),
                                       native=lambda **_: "native") == "native"


class _FakeHipTensor:
    """Just enough of a HIP tensor for block_eligible's shape checks."""

    def __init__(self, n):
        self.is_cuda = True
        self.dtype = torch.float32
        self.shape = (n, n, 128)
        self.device = torch.device("cpu")

    def dim(self):
        return 3

    def stride(self, d=None):
        s = (self.shape[1] * 128, 128, 1)
        return s if d is None else s[d]

    def element_size(self):
        return 4

    def data_ptr(self):
        return 0


def test_block_eligibility_bounds_the_pair_size():
    """N outside 1..4096 is rejected with a reason (the C ABI would return 2),
    so the registry falls back to native instead of raising."""
    m = _protenix_like()
    for n in (0, 4097, 5000):
        ok, reason = ta.block_eligible(m, _FakeHipTensor(n), None)
        assert not ok and reason == "N must lie in 1..4096", (n, reason)


class _TriangleAttentionModule(torch.nn.Module):
    """A Protenix-shaped module (weak-referenceable, like the real one)."""

    def __init__(self):
        super().__init__()
        self.layer_norm = torch.nn.LayerNorm(128)
        self.linear = torch.nn.Linear(128, 4, bias=False)
        self.mha = torch.nn.Module()
        for name in ("linear_q", "linear_k", "linear_v"):
            setattr(self.mha, name, torch.nn.Linear(128, 128, bias=False))
        self.mha.linear_g = torch.nn.Linear(128, 128)
        self.mha.linear_o = torch.nn.Linear(128, 128)
        self.mha.no_heads, self.mha.c_hidden, self.inf = 4, 32, 1e9


def test_packed_block_weights_are_cached_until_a_parameter_changes():
    m = _TriangleAttentionModule()
    first = ta._weights_of(m)
    assert ta._weights_of(m) is first  # no re-concatenation per call
    with torch.no_grad():
        m.mha.linear_k.weight.mul_(2.0)  # in place: the version counter moves
    second = ta._weights_of(m)
    assert second is not first
    assert torch.equal(second.w_qkvg[128:256], m.mha.linear_k.weight)
    m.mha.linear_o = torch.nn.Linear(128, 128)  # a new parameter object
    third = ta._weights_of(m)
    assert third is not second and torch.equal(third.w_o, m.mha.linear_o.weight)
    assert ta._weights_of(m) is third


def test_modules_built_under_inference_mode_are_packed_without_the_cache():
    """Parameters created under torch.inference_mode are inference tensors,
    which keep no version counter: the packed weights are rebuilt on every
    call (an in-place change under inference mode stays visible) and the
    eligibility check passes instead of raising."""
    with torch.inference_mode():
        m = _TriangleAttentionModule()
        first = ta._weights_of(m)
        assert torch.equal(first.w_qkvg[:128], m.mha.linear_q.weight)
        m.mha.linear_q.weight.mul_(3.0)
        second = ta._weights_of(m)
    assert second is not first
    assert torch.equal(second.w_qkvg[:128], m.mha.linear_q.weight)
    ok, reason = ta.block_eligible(m, _FakeHipTensor(8), None)  # weights and "z" on the CPU
    assert ok and reason == "", reason
