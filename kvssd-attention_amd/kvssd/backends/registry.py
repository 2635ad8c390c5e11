"""Attention backend registry (reference: src/kvssd/backends/registry.py:13-68).

Automatic selection on a GPU device tries ``hip`` then ``reference`` (the
reference tries ``cuda``, ``triton``, ``reference``); on any other device only
``reference``.  The choice is observable through ``backend.name``; an explicit
name fails closed with the backend's reason.  A ROCm GPU whose native library
is missing or stale is a broken install, not a capability difference, so
automatic selection raises there instead of quietly using ``reference``.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from .. import _native
from .base import AttentionBackend, BackendAvailability
from .hip import HipAttentionBackend
from .reference import ReferenceAttentionBackend
from .unavailable import CudaExtensionBackend, TritonAttentionBackend

BackendFactory = Callable[[], AttentionBackend]

_BUILTINS: dict[str, BackendFactory] = {
    "hip": HipAttentionBackend,
    "cuda": CudaExtensionBackend,
    "reference": ReferenceAttentionBackend,
    "triton": TritonAttentionBackend,
}
_GPU_ORDER = ("hip", "reference")


def register_attention_backend(name: str, factory: BackendFactory) -> None:
    key = name.strip().lower()
    if not key or key == "auto":
        raise ValueError("backend name must be non-empty and cannot be 'auto'")
    _BUILTINS[key] = factory


def available_attention_backends(device: str | torch.device) -> list[BackendAvailability]:
    target = torch.device(device)
    return [factory().probe(target) for factory in _BUILTINS.values()]


def resolve_attention_backend(
    requested: str | AttentionBackend | None,
    device: str | torch.device,
) -> AttentionBackend:
    target = torch.device(device)
    if requested is not None and not isinstance(requested, str):
        state = requested.probe(target)
        if not state.available:
            raise RuntimeError(f"attention backend '{state.name}' unavailable: {state.reason}")
        return requested
    key = (requested or "auto").strip().lower()
    if key == "auto":
        order = _GPU_ORDER if target.type == "cuda" else ("reference",)
        for name in order:
            factory = _BUILTINS.get(name)
            if factory is None:
                continue
            backend = factory()
            state = backend.probe(target)
            if state.available:
                return backend
            if name == "hip" and torch.version.hip is not None and torch.cuda.is_available():
                loaded, why = _native.available()
                if not loaded:
                    raise RuntimeError(f"attention backend 'hip' unavailable: {why}")
        raise RuntimeError(f"no attention backend is available for {target}")
    if key not in _BUILTINS:
        choices = ", ".join(["auto", *_BUILTINS])
        raise ValueError(f"unknown attention backend '{key}'; choose one of: {choices}")
    backend = _BUILTINS[key]()
    state = backend.probe(target)
    if not state.available:
        raise RuntimeError(f"attention backend '{key}' unavailable: {state.reason}")
    return backend
