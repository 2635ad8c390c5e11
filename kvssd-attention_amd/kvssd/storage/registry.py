"""Storage backend registry (reference: src/kvssd/storage/registry.py:12-66).

Automatic selection tries ``gds`` (never available on ROCm), then
``direct``, then ``buffered``; an explicit name fails closed with the backend's
reason.
"""

from __future__ import annotations

from collections.abc import Callable
from pathlib import Path

from .base import StorageAvailability, StorageBackend
from .buffered import BufferedStorageBackend
from .direct import DirectIOStorageBackend
from .gds import GDSStorageBackend

StorageFactory = Callable[[Path], StorageBackend]

_BUILTINS: dict[str, StorageFactory] = {
    "gds": GDSStorageBackend,
    "direct": DirectIOStorageBackend,
    "buffered": BufferedStorageBackend,
}
_AUTO_ORDER = ("gds", "direct", "buffered")


def register_storage_backend(name: str, factory: StorageFactory) -> None:
    key = name.strip().lower()
    if not key or key == "auto":
        raise ValueError("backend name must be non-empty and cannot be 'auto'")
    _BUILTINS[key] = factory


def available_storage_backends(path: str | Path) -> list[StorageAvailability]:
    target = Path(path)
    return [factory(target).probe() for factory in _BUILTINS.values()]


def resolve_storage_backend(requested: str | StorageBackend | None, path: str | Path) -> StorageBackend:
    target = Path(path)
    if requested is not None and not isinstance(requested, str):
        state = requested.probe()
        if not state.available:
            raise RuntimeError(f"storage backend '{state.name}' unavailable: {state.reason}")
        return requested
    key = (requested or "auto").strip().lower()
    if key == "auto":
        for name in _AUTO_ORDER:
            factory = _BUILTINS.get(name)
            if factory is None:
                continue
            backend = factory(target)
            if backend.probe().available:
                return backend
        raise RuntimeError(f"no storage backend is available for {target}")
    if key not in _BUILTINS:
        choices = ", ".join(["auto", *_BUILTINS])
        raise ValueError(f"unknown storage backend '{key}'; choose one of: {choices}")
    backend = _BUILTINS[key](target)
    state = backend.probe()
    if not state.available:
        raise RuntimeError(f"storage backend '{key}' unavailable: {state.reason}")
    return backend
