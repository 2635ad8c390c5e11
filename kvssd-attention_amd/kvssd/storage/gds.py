"""GPUDirect Storage placeholder.

The reference's cuFile tier (src/kvssd/storage/gds.py:13-97,
csrc/gds_bindings.cpp) needs NVIDIA's libcufile and has no ROCm counterpart
here.  The name stays registered so ``available_storage_backends`` keeps
the reference's shape and an explicit ``"gds"`` request fails closed with the
reason instead of silently changing the data path.
"""

from __future__ import annotations

from pathlib import Path

import torch

from ..format import BlockEntry
from .base import StorageAvailability

REASON = "GPUDirect Storage (cuFile) is NVIDIA-only and is not part of the ROCm build"


class GDSStorageBackend:
    name = "gds"

    def __init__(self, path: str | Path):
        self.path = Path(path)

    def probe(self) -> StorageAvailability:
        return StorageAvailability(self.name, False, True, True, REASON)

    def allocate_buffer(self, size: int, *, pinned: bool = False, device: torch.device | None = None) -> torch.Tensor:
        raise RuntimeError(REASON)

    def read_into(self, entry: BlockEntry, destination: torch.Tensor) -> None:
        raise RuntimeError(REASON)

    def close(self) -> None:
        pass
