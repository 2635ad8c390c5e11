"""Named backends chosen by probing: the one resolution procedure behind the
attention-backend registry (src/kvssd/backends/registry.py:23-68) and the
storage-backend registry (src/kvssd/storage/registry.py:22-66).

A registry maps lower-case names to factories.  ``resolve`` accepts an
instance (probed, returned if available), an explicit name (built, probed,
failing closed with the backend's own reason) or ``auto``/``None`` (the first
available name of an order that depends on the target).  The messages are the
reference's, since callers match on them.
"""

from __future__ import annotations

from collections.abc import Callable, Iterable
from typing import Any


class Registry:
    def __init__(
        self,
        kind: str,
        builtins: dict[str, Callable[..., Any]],
        *,
        build: Callable[[Callable[..., Any], Any], Any],
        probe: Callable[[Any, Any], Any],
        auto_order: Callable[[Any], Iterable[str]],
        veto: Callable[[str, Any, Any], None] | None = None,
    ):
        self.kind = kind
        self.factories = dict(builtins)
        self._build = build
        self._probe = probe
        self._auto_order = auto_order
        self._veto = veto

    def register(self, name: str, factory: Callable[..., Any]) -> None:
        key = name.strip().lower()
        if key in ("", "auto"):
            raise ValueError("backend name must be non-empty and cannot be 'auto'")
        self.factories[key] = factory

    def available(self, target: Any) -> list[Any]:
        return [self._probe(self._build(f, target), target) for f in self.factories.values()]

    def _unavailable(self, name: str, reason: str) -> RuntimeError:
        return RuntimeError(f"{self.kind} backend '{name}' unavailable: {reason}")

    def resolve(self, requested: Any, target: Any) -> Any:
        if requested is not None and not isinstance(requested, str):
            state = self._probe(requested, target)
            if not state.available:
                raise self._unavailable(state.name, state.reason)
            return requested
        key = (requested or "auto").strip().lower()
        if key != "auto":
            factory = self.factories.get(key)
            if factory is None:
                names = ", ".join(["auto", *self.factories])
                raise ValueError(f"unknown {self.kind} backend '{key}'; choose one of: {names}")
            backend = self._build(factory, target)
            state = self._probe(backend, target)
            if not state.available:
                raise self._unavailable(key, state.reason)
            return backend
        for name in self._auto_order(target):
            if name not in self.factories:
                continue
            backend = self._build(self.factories[name], target)
            state = self._probe(backend, target)
            if state.available:
                return backend
            if self._veto is not None:
                self._veto(name, state, target)
        raise RuntimeError(f"no {self.kind} backend is available for {target}")
