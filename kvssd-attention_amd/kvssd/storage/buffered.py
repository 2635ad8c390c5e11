"""Buffered positioned reads through the page cache (the reference's
``buffered`` backend, src/kvssd/storage/buffered.py:13-82).  Destinations may
be page-locked: the loader reads records straight into the pipeline's
staging rows."""

from __future__ import annotations

from pathlib import Path

import torch

from ..format import BlockEntry
from .base import StorageAvailability
from .posix import PositionedFile, destination_view


class BufferedStorageBackend(PositionedFile):
    name = "buffered"

    def __init__(self, path: str | Path):
        super().__init__(path)

    def probe(self) -> StorageAvailability:
        if self.path.is_file():
            return StorageAvailability(self.name, True, False, True, "portable buffered positioned reads")
        return StorageAvailability(self.name, False, False, True, f"data file does not exist: {self.path}")

    def allocate_buffer(self, size: int, *, pinned: bool = False, device: torch.device | None = None) -> torch.Tensor:
        return torch.empty(size, dtype=torch.uint8, pin_memory=bool(pinned) and torch.cuda.is_available())

    def read_into(self, entry: BlockEntry, destination: torch.Tensor) -> None:
        if destination.device.type != "cpu":
            raise ValueError("buffered backend requires a CPU destination tensor")
        if destination.dtype != torch.uint8 or destination.numel() < entry.length:
            raise ValueError("destination must be a sufficiently large uint8 tensor")
        got = self.read_exact(entry.offset, destination_view(destination, entry))
        if got != entry.length:
            raise EOFError(
                f"short read for layer={entry.layer}, block={entry.block}: expected {entry.length}, got {got}"
            )
