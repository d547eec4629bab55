"""Registry policy (fireprot_amd.registry), mirroring the reference's
tests/operators/test_registry.py and test_rust_registry.py plus the Rust
policy's ordering, cache and manifest rules (crates/fireprot-core/src/
registry.rs:96-259; bridge predicate marshalling lib.rs:23-57)."""
from __future__ import annotations

import pytest

from fireprot_amd.registry import OperationRegistry, OperationSignature


def _signature(**overrides) -> OperationSignature:
    values = {"operation": "triangle_multiplication", "device_type": "cuda",
              "architecture": "gfx950", "dtype": "float32", "shape": (124, 124, 128),
              "layout": "contiguous", "mode": "inference", "mask": "dense", "inplace": True}
    values.update(overrides)
    return OperationSignature.create(**values)


def test_registry_selects_highest_priority_supported_candidate():
    registry = OperationRegistry()
    registry.register(operation="triangle_multiplication", name="slow",
                      function=lambda value: f"slow:{value}", supports=lambda s: True, priority=1)
    registry.register(operation="triangle_multiplication", name="fast",
                      function=lambda value: f"fast:{value}",
                      supports=lambda s: s.architecture == "gfx950", priority=10)
    assert registry.dispatch(_signature(), lambda value: f"native:{value}", "x") == "fast:x"
    assert registry.manifest()["selection_counts"] == [
        {"operation": "triangle_multiplication", "implementation": "fast", "count": 1}]


def test_registry_falls_back_and_records_rejection_reason():
    registry = OperationRegistry()
    registry.register(operation="triangle_multiplication", name="gfx950-only",
                      function=lambda value: value,
                      supports=lambda s: (False, "architecture mismatch"))
    assert registry.dispatch(_signature(architecture="gfx942"), lambda: "native") == "native"
    decision = registry.manifest()["decisions"][0]
    assert decision["selected"] == "native"
    assert decision["rejected"] == [{"implementation": "gfx950-only",
                                     "reason": "architecture mismatch"}]


def test_registry_cache_is_invalidated_by_new_registration():
    registry = OperationRegistry()
    signature = _signature()
    assert registry.resolve(signature).implementation is None
    assert registry.resolve(signature).cache_hit is True
    registry.register(operation="triangle_multiplication", name="new", function=lambda: None,
                      supports=lambda s: True)
    selection = registry.resolve(signature)
    assert selection.cache_hit is False and selection.implementation.name == "new"
    assert registry.resolve(signature).cache_hit is True


def test_capability_error_fails_closed_to_native():
    registry = OperationRegistry()

    def broken(signature):
        raise RuntimeError("probe failed")

    registry.register(operation="triangle_multiplication", name="broken",
                      function=lambda: "wrong", supports=broken)
    assert registry.dispatch(_signature(), lambda: "native") == "native"
    reason = registry.manifest()["decisions"][0]["rejected"][0]["reason"]
    assert reason == "capability error: RuntimeError: probe failed"


def test_predicate_results_follow_bridge_semantics():
    registry = OperationRegistry()
    registry.register(operation="op", name="a-false", function=lambda: "a", supports=lambda s: 0,
                      priority=5)
    registry.register(operation="op", name="b-tuple3", function=lambda: "b",
                      supports=lambda s: (False, "x", "y"), priority=4)
    registry.register(operation="op", name="c-truthy", function=lambda: "c",
                      supports=lambda s: (1, "fine"), priority=3)
    assert registry.dispatch(_signature(operation="op"), lambda: "native") == "c"
    rejected = registry.manifest()["decisions"][0]["rejected"]
    assert rejected[0] == {"implementation": "a-false", "reason": "capability returned false"}
    assert rejected[1]["reason"].startswith("capability error: ValueError")


def test_ordering_ties_duplicates_and_unregister():
    registry = OperationRegistry()
    for name in ("zeta", "alpha"):
        registry.register(operation="op", name=name, function=lambda n=name: n,
                          supports=lambda s: True, priority=7)
    assert registry.dispatch(_signature(operation="op"), lambda: "native") == "alpha"
    with pytest.raises(ValueError):
        registry.register(operation="op", name="alpha", function=lambda: None,
                          supports=lambda s: True)
    with pytest.raises(TypeError):
        registry.register(operation="op", name="bad", function=None, supports=lambda s: True)
    registry.unregister("op", "alpha")
    assert registry.dispatch(_signature(operation="op"), lambda: "native") == "zeta"
    with pytest.raises(KeyError):
        registry.unregister("op", "alpha")
    names = [c["name"] for c in registry.manifest()["implementations"]["op"]]
    assert names == ["zeta"]


def test_cache_keys_on_strides_and_attributes_and_counts_survive():
    registry = OperationRegistry()
    seen = []
    registry.register(operation="op", name="x", function=lambda: "x",
                      supports=lambda s: seen.append(s) or True)
    a = _signature(operation="op", strides=(1, 2, 3))
    b = _signature(operation="op", strides=(3, 2, 1))
    c = _signature(operation="op", strides=(1, 2, 3), attributes={"k": 1})
    for sig in (a, a, b, c):
        registry.resolve(sig)
    assert len(seen) == 3
    assert registry.count("op", "x") == 4
    registry.register(operation="op", name="y", function=lambda: "y", supports=lambda s: False)
    assert registry.count("op", "x") == 4          # history survives registration
    registry.clear_runtime_state()
    assert registry.count("op", "x") == 0 and registry.manifest()["decisions"] == []


def test_signature_from_tensor_records_layout_and_strides():
    import torch

    from fireprot_amd.registry import signature_from_tensor

    t = torch.empty(4, 5, 6).transpose(0, 1)
    sig = signature_from_tensor("op", t, architecture="cpu", mode="inference", mask="none",
                                inplace=False, attributes={"b": 2, "a": 1})
    assert sig.layout == "strided" and sig.strides == tuple(t.stride())
    assert sig.attributes == (("a", "1"), ("b", "2")) and sig.dtype == "float32"
