"""Scope isolation, source pinning and native fallback of the OpenFold3
``_attention`` consumer on the CPU (mirrors the reference's
tests/operators/test_openfold3_attention_scope.py)."""
from __future__ import annotations

import hashlib
import importlib.util
from concurrent.futures import ThreadPoolExecutor
from contextvars import copy_context
from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import openfold3 as of3


def test_scope_isolates_other_threads_and_restores_original():
    native = lambda x: ("native", x)  # noqa: E731
    target = SimpleNamespace(_attention=native)
    selected = lambda original, x: ("selected", x)  # noqa: E731
    with ThreadPoolExecutor(max_workers=1) as pool:
        with of3._scoped_hook(target, selected):
            assert target._attention(1) == ("selected", 1)
            assert pool.submit(target._attention, 2).result() == ("native", 2)
            leaked = target._attention
            inherited = copy_context()
        assert target._attention is native
        assert leaked(3) == ("native", 3)
        assert inherited.run(leaked, 4) == ("native", 4)


def test_nested_and_concurrent_installs_rejected_without_displacing_outer():
    target = SimpleNamespace(_attention=lambda: "native")

    def attempt():
        with of3._scoped_hook(target, lambda original: "inner"):
            pytest.fail("a second installation was accepted")

    with of3._scoped_hook(target, lambda original: "outer"):
        with pytest.raises(RuntimeError, match="already installed"):
            attempt()
        with ThreadPoolExecutor(max_workers=1) as pool:
            with pytest.raises(RuntimeError, match="already installed"):
                pool.submit(attempt).result()
        assert target._attention() == "outer"
    assert target._attention() == "native"


def test_exception_cleanup_and_external_replacement_detection():
    native = lambda: "native"  # noqa: E731
    target = SimpleNamespace(_attention=native)
    with pytest.raises(ValueError, match="model failure"):
        with of3._scoped_hook(target, lambda original: "selected"):
            raise ValueError("model failure")
    assert target._attention is native
    foreign = lambda: "foreign"  # noqa: E731
    with pytest.raises(RuntimeError, match="changed during"):
        with of3._scoped_hook(target, lambda original: "selected"):
            target._attention = foreign
    assert target._attention is foreign
    # the failed cleanup released the guard without displacing the foreign owner
    with of3._scoped_hook(target, lambda original: original()):
        assert target._attention() == "foreign"


def _module_from(tmp_path, text):
    path = tmp_path / "attention.py"
    path.write_text(text)
    spec = importlib.util.spec_from_file_location("of3_attention_under_test", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module, hashlib.sha256(path.read_bytes()).hexdigest()


def test_attention_scope_pins_source_and_original_function(tmp_path, monkeypatch):
    module, digest = _module_from(
        tmp_path, "def _attention(q, k, v, biases, use_high_precision=False):\n    return 'native'\n")
    with pytest.raises(RuntimeError, match="Unsupported OpenFold3 attention source"):
        with of3.attention_scope(lambda original, *a, **k: "selected", module):
            pass
    monkeypatch.setattr(of3, "SOURCE_SHA256", digest)
    with of3.attention_scope(lambda original, *a, **k: "selected", module):
        assert module._attention(1, 2, 3, []) == "selected"
    assert module._attention(1, 2, 3, []) == "native"
    module._attention = lambda *a, **k: "foreign"
    with pytest.raises(RuntimeError, match="already replaced"):
        with of3.attention_scope(lambda original, *a, **k: "selected", module):
            pass


def test_native_fallback_without_kernel_preserves_call_arguments():
    dispatcher = of3.AttentionDispatcher(None)
    query = torch.zeros(1, 4, 3, 32)
    biases = [torch.zeros(1, 1, 1, 3), torch.zeros(1, 4, 3, 3)]
    calls = []

    def native(q, k, v, b, use_high_precision=False):
        calls.append((q, k, v, b, use_high_precision))
        return q

    with torch.no_grad():
        for _ in range(2):
            assert dispatcher(native, query, query, query, biases, True) is query
    assert len(calls) == 2 and all(c[3] is biases and c[4] is True for c in calls)
    report = dispatcher.manifest()
    assert report["kernel"] is None and report["launches_submitted"] == 0
    assert all(d["selected"] == "native" for d in report["registry"]["decisions"])
    reasons = {r["reason"] for d in report["registry"]["decisions"] for r in d["rejected"]}
    assert reasons == {"no HIP kernel"}


def test_ineligible_tensors_go_native_with_reason():
    kernel = SimpleNamespace(device=0, receipt={}, launches_submitted=0)
    dispatcher = of3.AttentionDispatcher(kernel)
    q = torch.zeros(2, 4, 8, 32)
    biases = [torch.zeros(2, 1, 1, 8), torch.zeros(1, 4, 8, 8)]
    native = lambda q, k, v, b, use_high_precision=False: "native"  # noqa: E731
    with torch.no_grad():
        assert dispatcher(native, q, q, q, biases) == "native"
    assert dispatcher(native, q, q, q, biases) == "native"  # grad enabled
    # a non-tensor query bypasses the registry entirely
    assert dispatcher(native, "q", q, q, biases) == "native"
    decisions = dispatcher.manifest()["registry"]["decisions"]
    assert len(decisions) == 2
    modes = {d["signature"]["mode"] for d in decisions}
    assert modes == {"inference", "training"}


def test_tensor_contract_reasons():
    q = torch.zeros(2, 4, 8, 32)
    biases = [torch.zeros(2, 1, 1, 8), torch.zeros(1, 4, 8, 8)]
    assert of3.tensor_contract(q, q, q, biases)[1] == "autograd is enabled"
    with torch.no_grad():
        assert "biases" in of3.tensor_contract(q, q, q, biases[:1])[1]
        assert "plain tensors" in of3.tensor_contract(q, q, q, [biases[0], None])[1]
        assert "HIP device" in of3.tensor_contract(q, q, q, biases)[1]
