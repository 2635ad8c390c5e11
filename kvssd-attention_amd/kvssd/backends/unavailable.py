"""Backend names of the reference that have no MI355X implementation.

``cuda`` (the torch extension kvssd._C, src/kvssd/backends/cuda.py) and
``triton`` (src/kvssd/backends/triton.py) stay registered so
``available_attention_backends`` lists them with the reason, and an explicit
request fails closed (src/kvssd/backends/registry.py:60-68) instead of
silently running something else.  The fused kernel on ROCm is ``hip``.
"""

from __future__ import annotations

import torch

from .base import BackendAvailability, PackedBatch


class CudaExtensionBackend:
    name = "cuda"

    def probe(self, device: torch.device) -> BackendAvailability:
        device = torch.device(device)
        if device.type != "cuda":
            reason = f"CUDA extension requires a CUDA device, got {device.type}"
        else:
            reason = "the CUDA extension kvssd._C is replaced by the 'hip' backend on ROCm"
        return BackendAvailability(self.name, False, True, False, reason, device.type)

    def run(self, query: torch.Tensor, batch: PackedBatch, sm_scale: float):
        raise RuntimeError(self.probe(query.device).reason)


class TritonAttentionBackend:
    name = "triton"

    def probe(self, device: torch.device) -> BackendAvailability:
        device = torch.device(device)
        reason = "Triton dispatch is not part of the MI355X build; use the 'hip' backend"
        return BackendAvailability(self.name, False, True, False, reason, device.type)

    def run(self, query: torch.Tensor, batch: PackedBatch, sm_scale: float):
        raise RuntimeError(self.probe(query.device).reason)
