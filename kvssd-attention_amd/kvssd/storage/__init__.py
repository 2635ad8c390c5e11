"""Storage backend contracts and built-in implementations (host-side reads)."""

from .base import StorageAvailability, StorageBackend
from .registry import available_storage_backends, register_storage_backend, resolve_storage_backend

__all__ = [
    "StorageAvailability",
    "StorageBackend",
    "available_storage_backends",
    "register_storage_backend",
    "resolve_storage_backend",
]
