"""The module-level installers (fireprot_amd.hooks) on stand-in classes.

Protenix and AtlasFold are not importable here, so the tests build classes
with their attribute layout (patches/protenix/0005-*.patch:14-48;
adapters/atlasfold/runtime.py:32-71) and pass them in.  What is checked:
the hooks route calls through the block dispatch and fall back to the
original forward with the same arguments when the block cannot serve (here:
CPU tensors), installation is idempotent and reversible, and the refusals of
the reference's AtlasFold runtime (runtime.py:140-157) hold: an already
wrapped forward, an instance forward, a class method replaced from another
source file, a second install, a model in training mode.
"""
from __future__ import annotations

import functools

import pytest
import torch

from fireprot_amd import hooks
from fireprot_amd import triangle_attention as ta
from fireprot_amd.registry import registry


class _Attention(torch.nn.Module):
    def __init__(self):
        super().__init__()
        for name in ("linear_q", "linear_k", "linear_v"):
            setattr(self, name, torch.nn.Linear(128, 128, bias=False))
        self.linear_g = torch.nn.Linear(128, 128)
        self.linear_o = torch.nn.Linear(128, 128)
        self.no_heads, self.c_hidden = 4, 32


class TriangleAttention(torch.nn.Module):
    """Protenix's TriangleAttention attribute layout; forward records its call."""

    def __init__(self, starting=True):
        super().__init__()
        self.starting = starting
        self.layer_norm = torch.nn.LayerNorm(128)
        self.linear = torch.nn.Linear(128, 4, bias=False)
        self.mha = _Attention()
        self.inf = 1e9
        self.calls = []

    def forward(self, x, mask=None, chunk_size=None, inplace_safe=False):
        self.calls.append((x, mask, chunk_size, inplace_safe))
        return torch.full_like(x, 7.0)


class StartingNode(torch.nn.Module):
    """AtlasFold's triangle node layout; forward(z, mask, kernel_backend)."""

    def __init__(self):
        super().__init__()
        self.layernorm = torch.nn.LayerNorm(128)
        self.linear_qkv = torch.nn.Linear(128, 384, bias=False)
        self.linear_bias = torch.nn.Linear(128, 4, bias=False)
        self.linear_g = torch.nn.Linear(128, 128, bias=False)
        self.linear_out = torch.nn.Linear(128, 128, bias=False)
        self.num_heads, self.channel_hidden, self.inf = 4, 32, 1e9
        self.scale = 32 ** -0.5
        self.calls = []

    def forward(self, z, mask, kernel_backend="torch"):
        self.calls.append(kernel_backend)
        return torch.full_like(z, 3.0)


class EndingNode(StartingNode):
    pass


class _Model(torch.nn.Module):
    def __init__(self):
        super().__init__()
        self.start = StartingNode()
        self.end = EndingNode()
        self.other = torch.nn.Linear(4, 4)


@pytest.fixture
def protenix_cls():
    """A fresh subclass per test, so installs never leak between tests."""
    cls = type("TriangleAttention", (TriangleAttention,), {"forward": TriangleAttention.forward})
    yield cls
    if hooks.protenix_manifest()["installed"]:
        hooks.uninstall_protenix()


def test_protenix_install_routes_through_the_block_dispatch_and_falls_back(protenix_cls):
    original = protenix_cls.forward
    manifest = hooks.install_protenix(protenix_cls)
    assert manifest["installed"] and manifest["hooks"] == ["TriangleAttention.forward"]
    assert protenix_cls.forward is not original and protenix_cls.forward.__wrapped__ is original
    assert hooks.install_protenix(protenix_cls)["installed"]  # idempotent
    registry.clear_runtime_state()
    for starting in (True, False):
        m = protenix_cls(starting=starting).eval()
        x, mask = torch.randn(6, 6, 128), torch.ones(6, 6)
        with torch.inference_mode():
            out = m(x, mask, chunk_size=4, inplace_safe=True)
        assert torch.equal(out, torch.full_like(x, 7.0))  # the original forward ran
        assert m.calls == [(x, mask, 4, True)]            # with the caller's arguments
    decisions = registry.manifest()["decisions"]
    assert {d["signature"]["attributes"]["ending"] for d in decisions} == {"True", "False"}
    assert all(d["selected"] == "native" for d in decisions)
    assert all(r["reason"] == "device is not CUDA/HIP" for d in decisions for r in d["rejected"])
    hooks.uninstall_protenix()
    assert protenix_cls.forward is original
    assert not hooks.protenix_manifest()["installed"]


def test_protenix_batched_input_keeps_its_shape_on_fallback(protenix_cls):
    hooks.install_protenix(protenix_cls)
    m = protenix_cls().eval()
    x = torch.randn(1, 5, 5, 128)
    with torch.inference_mode():
        out = m(x, torch.ones(1, 5, 5, dtype=torch.bool))
    assert out.shape == x.shape and m.calls[0][0] is x


def test_protenix_refuses_wrapped_and_foreign_forwards(protenix_cls):
    @functools.wraps(TriangleAttention.forward)
    def wrapped(self, x, mask=None, **kwargs):
        return TriangleAttention.forward(self, x, mask, **kwargs)

    cls = type("TriangleAttention", (TriangleAttention,), {"forward": wrapped})
    with pytest.raises(ValueError, match="already modified"):
        hooks.install_protenix(cls)
    namespace: dict = {}
    exec(compile("def forward(self, x, mask=None):\n    return x\n", "<elsewhere>", "exec"),
         namespace)
    cls = type("TriangleAttention", (TriangleAttention,), {"forward": namespace["forward"]})
    with pytest.raises(ValueError, match="replaced triangle class method"):
        hooks.install_protenix(cls)
    assert not hooks.protenix_manifest()["installed"]
    hooks.install_protenix(protenix_cls)
    with pytest.raises(ValueError, match="another class"):
        hooks.install_protenix(cls)


def test_protenix_uninstall_refuses_a_hook_replaced_since(protenix_cls):
    hooks.install_protenix(protenix_cls)
    hooked = protenix_cls.forward
    protenix_cls.forward = lambda self, x, mask=None: x
    with pytest.raises(ValueError, match="replaced after install"):
        hooks.uninstall_protenix()
    protenix_cls.forward = hooked
    hooks.uninstall_protenix()


def test_atlasfold_hooks_are_per_instance_and_reversible():
    model = _Model().eval()
    h = hooks.AtlasFoldHooks(model, starting_cls=StartingNode, ending_cls=EndingNode)
    assert "forward" in model.start.__dict__ and "forward" in model.end.__dict__
    assert "forward" not in model.other.__dict__
    assert StartingNode.forward is StartingNode.__dict__["forward"]  # class untouched
    z = torch.randn(1, 6, 6, 128)
    mask = torch.ones(1, 6, 6, dtype=torch.bool)
    registry.clear_runtime_state()
    with torch.inference_mode():
        assert torch.equal(model.start(z, mask), torch.full_like(z, 3.0))
        assert torch.equal(model.end(z, mask, "cuequivariance"), torch.full_like(z, 3.0))
    assert model.start.calls == ["torch"] and model.end.calls == ["cuequivariance"]
    assert h.counts == {"dispatched": 1, "kept": 1}
    decision = registry.manifest()["decisions"][0]
    assert decision["signature"]["operation"] == ta.BLOCK_OPERATION
    assert decision["selected"] == "native"
    with pytest.raises(ValueError, match="already installed"):
        hooks.AtlasFoldHooks(model, starting_cls=StartingNode, ending_cls=EndingNode)
    h.uninstall()
    assert "forward" not in model.start.__dict__ and "forward" not in model.end.__dict__
    assert not hasattr(model, hooks.AtlasFoldHooks.ATTRIBUTE)
    hooks.AtlasFoldHooks(model, starting_cls=StartingNode, ending_cls=EndingNode).uninstall()


def test_atlasfold_refusals_change_nothing():
    model = _Model().eval()
    model.end.forward = lambda z, mask, kernel_backend="torch": z  # an instance override
    with pytest.raises(ValueError, match="already modified"):
        hooks.AtlasFoldHooks(model, starting_cls=StartingNode, ending_cls=EndingNode)
    assert "forward" not in model.start.__dict__  # refused before any change
    del model.end.forward
    model.train()
    with pytest.raises(ValueError, match="eval mode"):
        hooks.AtlasFoldHooks(model, starting_cls=StartingNode, ending_cls=EndingNode)


def test_block_eligibility_rejects_hooked_layers_and_other_q_scales():
    """The fused block would skip a layer's forward hooks or precision
    override, and a q scale other than 1/sqrt(32) changes the arithmetic."""
    m = StartingNode().eval()

    class _Hip:  # just enough of a HIP tensor for the shape checks
        is_cuda, dtype, shape, device = True, torch.float32, (8, 8, 128), torch.device("cpu")

        def dim(self):
            return 3

        def stride(self, d=None):
            s = (1024, 128, 1)
            return s if d is None else s[d]

        def element_size(self):
            return 4

        def data_ptr(self):
            return 0

    assert ta.block_eligible(m, _Hip(), None) == (True, "")
    handle = m.linear_qkv.register_forward_hook(lambda *args: None)
    ok, reason = ta.block_eligible(m, _Hip(), None)
    assert not ok and "hooks" in reason
    handle.remove()
    m.linear_qkv.precision = torch.float32
    assert not ta.block_eligible(m, _Hip(), None)[0]
    m.linear_qkv.precision = None
    m.scale = 0.25
    assert ta.block_eligible(m, _Hip(), None) == (False, "module q scale is not 1/sqrt(32)")


def test_precision_override_read_as_attribute_lookup_does():
    """A ``precision`` defined by a layer's class (a value or a property)
    counts as the attribute lookup resolves it; an instance value counts; a
    class value of None or none at all lets the block run."""
    class _Hip:
        is_cuda, dtype, shape, device = True, torch.float32, (8, 8, 128), torch.device("cpu")

        def dim(self):
            return 3

        def stride(self, d=None):
            s = (1024, 128, 1)
            return s if d is None else s[d]

        def element_size(self):
            return 4

        def data_ptr(self):
            return 0

    m = StartingNode().eval()
    linear = m.linear_qkv
    base = type(linear)
    for attrs, expected in (({"precision": None}, True),
                            ({"precision": torch.float64}, False),
                            ({"precision": property(lambda self: None)}, True),
                            ({"precision": property(lambda self: torch.float64)}, False)):
        linear.__class__ = type("Linear", (base,), attrs)
        assert ta.block_eligible(m, _Hip(), None)[0] is expected, attrs
    linear.__class__ = base
    linear.precision = torch.bfloat16
    assert not ta.block_eligible(m, _Hip(), None)[0]
    del linear.precision
    assert ta.block_eligible(m, _Hip(), None) == (True, "")
