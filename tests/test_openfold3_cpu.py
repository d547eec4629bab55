"""Scope rules, source pinning and native fallback of the OpenFold3
``_attention`` consumer, on the CPU.

The scope rules are those the reference's adapter promises
(python/fireprot/adapters/openfold3/attention.py:43-84): one scope at a time,
only the opening context (and contexts copied from it) reaches the
dispatcher, stale references fall back to native, a foreign replacement is
reported and left in place.
"""
from __future__ import annotations

import asyncio
import hashlib
import importlib.util
import threading
from contextvars import copy_context
from types import SimpleNamespace

import pytest
import torch

from fireprot_amd import openfold3 as of3


def _recording_target():
    """A stand-in module whose native ``_attention`` records its callers."""
    seen = []

    def native(tag):
        seen.append(("native", tag))
        return "native"

    return SimpleNamespace(_attention=native), seen


def test_only_the_opening_context_reaches_the_dispatcher():
    target, seen = _recording_target()
    native = target._attention
    routed = []

    def dispatcher(original, tag):
        routed.append(tag)
        return original(f"via-{tag}")

    results = {}

    def worker(tag):
        results[tag] = target._attention(tag)

    with of3.ScopedAttentionHook(target, dispatcher) as hook:
        assert target._attention is hook and hook.native is native
        assert target._attention("main") == "native"
        # a thread started inside the scope runs in a fresh context: native
        thread = threading.Thread(target=worker, args=("thread",))
        thread.start()
        thread.join()
        # a context copied inside the scope inherits the active hook
        copied = copy_context()
        assert copied.run(target._attention, "copied") == "native"

        # an asyncio task copies the context of the code that creates it
        async def task():
            return target._attention("task")
        assert asyncio.run(task()) == "native"
        stale = target._attention
    assert routed == ["main", "copied", "task"]
    assert ("native", "thread") in seen and results["thread"] == "native"
    # after the scope: the module holds the native function again, and both a
    # stale reference and a context copied during the scope go native
    assert target._attention is native
    routed.clear()
    assert stale("late") == "native" and copied.run(stale, "late-copy") == "native"
    assert routed == []


def test_a_second_scope_is_refused_while_one_is_open():
    target, _ = _recording_target()
    other, _ = _recording_target()
    errors = []

    def contender():
        try:
            with of3.ScopedAttentionHook(other, lambda original, tag: "second"):
                pass
        except RuntimeError as error:
            errors.append(str(error))

    with of3.ScopedAttentionHook(target, lambda original, tag: "first"):
        # the slot is process-wide: another module or another thread is refused
        with pytest.raises(RuntimeError, match="already installed"):
            with of3.ScopedAttentionHook(target, lambda original, tag: "nested"):
                pass
        thread = threading.Thread(target=contender)
        thread.start()
        thread.join()
        assert errors and "already installed" in errors[0]
        assert target._attention("x") == "first"
        assert not isinstance(other._attention, of3.ScopedAttentionHook)
    # released: a new scope opens normally
    with of3.ScopedAttentionHook(other, lambda original, tag: "again"):
        assert other._attention("y") == "again"


def test_errors_inside_the_scope_and_foreign_replacements():
    target, _ = _recording_target()
    native = target._attention
    with pytest.raises(KeyError, match="lookup inside the model"):
        with of3.ScopedAttentionHook(target, lambda original, tag: "hooked"):
            raise KeyError("lookup inside the model")
    assert target._attention is native
    # a caller that swaps _attention itself while the scope is open keeps it
    def foreign(tag):
        return "foreign"

    with pytest.raises(RuntimeError, match="changed during its scope"):
        with of3.ScopedAttentionHook(target, lambda original, tag: "hooked"):
            target._attention = foreign
    assert target._attention is foreign
    # and the slot was released: the next scope wraps the foreign function
    with of3.ScopedAttentionHook(target, lambda original, tag: original(tag) + "+hooked"):
        assert target._attention("z") == "foreign+hooked"
    assert target._attention is foreign


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
