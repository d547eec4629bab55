"""Capability registry with native fallback, the reference operator surface.

Same public API as the reference's ``fireprot.ops.registry``
(python/fireprot/ops/registry.py:18-203): ``OperationSignature``,
``OperationRegistry.register/unregister/resolve/dispatch/manifest/
clear_runtime_state``, the module-level ``registry`` and
``signature_from_tensor``.  The reference delegates the policy to a Rust core
over PyO3 (crates/fireprot-core/src/registry.rs:96-259); no Rust toolchain is
part of this build, so the same policy is stated here in Python:

* candidates are ordered by priority (descending), then name, then version
  (registry.rs:118-124); names are unique per operation and registration
  clears the decision cache (registry.rs:109-126);
* resolution asks each candidate's ``supports(signature)`` in that order; the
  first ``True`` wins, ``(False, reason)`` records a rejection, and a raising
  predicate is a rejection ``"capability error: <Type>: <message>"`` -- it
  never selects unchecked code (registry.rs:173-190; bridge lib.rs:23-57);
* no match means the caller's native function (registry.py:151-164);
* decisions are cached per exact signature (shape, strides and attributes
  included) and every resolution counts toward ``selection_counts``; the
  manifest keeps the last decision per signature (registry.rs:150-259).
"""
from __future__ import annotations

import dataclasses
import threading
from collections.abc import Callable, Mapping
from typing import Any

Capability = Callable[["OperationSignature"], "bool | tuple[bool, str]"]
ImplementationFunction = Callable[..., Any]


@dataclasses.dataclass(frozen=True, slots=True)
class OperationSignature:
    operation: str
    device_type: str
    architecture: str
    dtype: str
    shape: tuple[int, ...]
    layout: str
    mode: str
    mask: str
    inplace: bool
    attributes: tuple[tuple[str, str], ...] = ()
    strides: tuple[int, ...] = ()

    @classmethod
    def create(cls, *, operation: str, device_type: str, architecture: str, dtype: str,
               shape, layout: str = "contiguous", mode: str = "inference",
               mask: str = "none", inplace: bool = False,
               attributes: Mapping[str, Any] | None = None, strides=()) -> "OperationSignature":
        normalized = tuple(sorted((str(k), str(v)) for k, v in (attributes or {}).items()))
        return cls(operation=operation, device_type=device_type, architecture=architecture,
                   dtype=dtype, shape=tuple(int(v) for v in shape), layout=layout, mode=mode,
                   mask=mask, inplace=bool(inplace), attributes=normalized,
                   strides=tuple(int(v) for v in strides))

    def as_dict(self) -> dict[str, Any]:
        result = dataclasses.asdict(self)
        result["shape"] = list(self.shape)
        result["strides"] = list(self.strides)
        result["attributes"] = dict(self.attributes)
        return result


@dataclasses.dataclass(frozen=True, slots=True)
class OperationImplementation:
    operation: str
    name: str
    function: ImplementationFunction
    supports: Capability
    priority: int
    version: str


@dataclasses.dataclass(frozen=True, slots=True)
class Selection:
    implementation: OperationImplementation | None
    rejected: tuple[tuple[str, str], ...]
    cache_hit: bool


class OperationRegistry:
    """Thread-safe registry whose missing match always means native fallback."""

    def __init__(self) -> None:
        self._candidates: dict[str, list[OperationImplementation]] = {}
        self._cache: dict[OperationSignature, Selection] = {}
        self._counts: dict[tuple[str, str], int] = {}
        self._decisions: dict[OperationSignature, Selection] = {}
        self._lock = threading.RLock()

    def register(self, *, operation: str, name: str, function: ImplementationFunction,
                 supports: Capability, priority: int = 0,
                 version: str = "1") -> OperationImplementation:
        if not callable(function) or not callable(supports):
            raise TypeError("function and supports must be callable")
        if not str(operation).strip() or not str(name).strip() or not str(version).strip():
            raise ValueError("operation, name and version must be non-empty")
        implementation = OperationImplementation(operation=operation, name=name,
                                                 function=function, supports=supports,
                                                 priority=int(priority), version=str(version))
        with self._lock:
            candidates = self._candidates.setdefault(operation, [])
            if any(c.name == name for c in candidates):
                raise ValueError(f"duplicate implementation {operation}/{name}")
            candidates.append(implementation)
            candidates.sort(key=lambda c: (-c.priority, c.name, c.version))
            self._cache.clear()
        return implementation

    def unregister(self, operation: str, name: str) -> None:
        with self._lock:
            candidates = self._candidates.get(operation, [])
            for index, candidate in enumerate(candidates):
                if candidate.name == name:
                    del candidates[index]
                    self._cache.clear()
                    return
            raise KeyError(f"unknown implementation {operation}/{name}")

    def resolve(self, signature: OperationSignature) -> Selection:
        with self._lock:
            cached = self._cache.get(signature)
            if cached is not None:
                result = dataclasses.replace(cached, cache_hit=True)
            else:
                chosen = None
                rejected: list[tuple[str, str]] = []
                for candidate in self._candidates.get(signature.operation, []):
                    try:
                        supported, reason = _verdict(candidate.supports(signature))
                    except Exception as error:  # a broken predicate fails closed
                        supported = False
                        reason = f"capability error: {type(error).__name__}: {error}"
                    if supported:
                        chosen = candidate
                        break
                    rejected.append((candidate.name, reason))
                result = Selection(chosen, tuple(rejected), False)
                self._cache[signature] = result
            name = result.implementation.name if result.implementation else "native"
            key = (signature.operation, name)
            self._counts[key] = self._counts.get(key, 0) + 1
            self._decisions[signature] = result
            return result

    def dispatch(self, signature: OperationSignature, fallback: ImplementationFunction,
                 *args: Any, **kwargs: Any) -> Any:
        selection = self.resolve(signature)
        function = (selection.implementation.function
                    if selection.implementation is not None else fallback)
        return function(*args, **kwargs)

    def count(self, operation: str, implementation: str) -> int:
        with self._lock:
            return self._counts.get((operation, implementation), 0)

    def manifest(self) -> dict[str, Any]:
        with self._lock:
            return {
                "implementations": {
                    operation: [{"name": c.name, "priority": c.priority, "version": c.version}
                                for c in candidates]
                    for operation, candidates in sorted(self._candidates.items())
                },
                "selection_counts": [
                    {"operation": op, "implementation": name, "count": count}
                    for (op, name), count in sorted(self._counts.items())
                ],
                "decisions": [
                    {"signature": sig.as_dict(),
                     "selected": sel.implementation.name if sel.implementation else "native",
                     "rejected": [{"implementation": n, "reason": r} for n, r in sel.rejected]}
                    for sig, sel in self._decisions.items()
                ],
                "policy_engine": {"language": "python", "module": __name__},
            }

    def clear_runtime_state(self) -> None:
        with self._lock:
            self._cache.clear()
            self._counts.clear()
            self._decisions.clear()


def _verdict(value: Any) -> tuple[bool, str]:
    """Interpret a predicate result as the reference bridge does (lib.rs:23-57).

    A 2-tuple is ``(truthy, reason)``; any other tuple length is an error;
    anything else is judged by truthiness with the reason "capability
    returned false".
    """
    if isinstance(value, tuple):
        if len(value) != 2:
            raise ValueError("capability tuple must have two items")
        return bool(value[0]), str(value[1])
    return bool(value), "capability returned false"


registry = OperationRegistry()


def signature_from_tensor(operation: str, tensor: Any, *, architecture: str, mode: str,
                          mask: str, inplace: bool,
                          attributes: Mapping[str, Any] | None = None) -> OperationSignature:
    layout = "contiguous" if tensor.is_contiguous() else "strided"
    return OperationSignature.create(
        operation=operation, device_type=tensor.device.type, architecture=architecture,
        dtype=str(tensor.dtype).removeprefix("torch."), shape=tuple(tensor.shape),
        strides=tuple(tensor.stride()), layout=layout, mode=mode, mask=mask, inplace=inplace,
        attributes=attributes)
