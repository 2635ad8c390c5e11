"""Storage-backend registry: the reference's public functions
(src/kvssd/storage/registry.py:22-66) over the shared probe-based resolver
(kvssd/_registry.py).

``auto`` tries ``gds`` (never available on ROCm), then ``direct`` (O_DIRECT),
then ``buffered``; an explicit name fails closed with the backend's reason.
"""

from __future__ import annotations

from collections.abc import Callable
from pathlib import Path

from .._registry import Registry
from .base import StorageAvailability, StorageBackend
from .buffered import BufferedStorageBackend
from .direct import DirectIOStorageBackend
from .gds import GDSStorageBackend

StorageFactory = Callable[[Path], StorageBackend]

_REGISTRY = Registry(
    "storage",
    {"gds": GDSStorageBackend, "direct": DirectIOStorageBackend, "buffered": BufferedStorageBackend},
    build=lambda factory, path: factory(path),
    probe=lambda backend, path: backend.probe(),
    auto_order=lambda path: ("gds", "direct", "buffered"),
)


def register_storage_backend(name: str, factory: StorageFactory) -> None:
    _REGISTRY.register(name, factory)


def available_storage_backends(path: str | Path) -> list[StorageAvailability]:
    return _REGISTRY.available(Path(path))


def resolve_storage_backend(requested: str | StorageBackend | None, path: str | Path) -> StorageBackend:
    return _REGISTRY.resolve(requested, Path(path))
