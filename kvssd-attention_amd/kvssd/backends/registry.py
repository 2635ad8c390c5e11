"""Attention-backend registry: the reference's public functions
(src/kvssd/backends/registry.py:23-68) over the shared probe-based resolver
(kvssd/_registry.py).

``auto`` on a GPU device tries ``hip`` then ``reference`` (the reference tries
``cuda``, ``triton``, ``reference``); on any other device only ``reference``.
The chosen backend reports itself through ``backend.name``.  A ROCm GPU whose
native library is missing or stale is a broken install, not a capability
difference, so ``auto`` raises there rather than quietly taking ``reference``.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from .. import _native
from .._registry import Registry
from .base import AttentionBackend, BackendAvailability
from .hip import HipAttentionBackend
from .reference import ReferenceAttentionBackend
from .unavailable import CudaExtensionBackend, TritonAttentionBackend

BackendFactory = Callable[[], AttentionBackend]


def _auto_order(device: torch.device) -> tuple[str, ...]:
    return ("hip", "reference") if device.type == "cuda" else ("reference",)


def _broken_install(name: str, state: BackendAvailability, device: torch.device) -> None:
    if name == "hip" and torch.version.hip is not None and torch.cuda.is_available():
        loaded, why = _native.available()
        if not loaded:
            raise RuntimeError(f"attention backend 'hip' unavailable: {why}")


_REGISTRY = Registry(
    "attention",
    {
        "hip": HipAttentionBackend,
        "cuda": CudaExtensionBackend,
        "reference": ReferenceAttentionBackend,
        "triton": TritonAttentionBackend,
    },
    build=lambda factory, device: factory(),
    probe=lambda backend, device: backend.probe(device),
    auto_order=_auto_order,
    veto=_broken_install,
)


def register_attention_backend(name: str, factory: BackendFactory) -> None:
    _REGISTRY.register(name, factory)


def available_attention_backends(device: str | torch.device) -> list[BackendAvailability]:
    return _REGISTRY.available(torch.device(device))


def resolve_attention_backend(requested: str | AttentionBackend | None, device: str | torch.device) -> AttentionBackend:
    return _REGISTRY.resolve(requested, torch.device(device))
