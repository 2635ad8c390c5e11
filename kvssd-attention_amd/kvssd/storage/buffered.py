"""Portable positioned reads (reference: src/kvssd/storage/buffered.py:13-82)."""

from __future__ import annotations

import os
import threading
from pathlib import Path

import torch

from ..format import BlockEntry
from .base import StorageAvailability


def host_buffer(size: int, pinned: bool) -> torch.Tensor:
    """A CPU uint8 buffer; page-locked when asked and a GPU runtime is present."""
    return torch.empty(size, dtype=torch.uint8, pin_memory=pinned and torch.cuda.is_available())


class BufferedStorageBackend:
    """Positioned reads into CPU tensors through the page cache."""

    name = "buffered"

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._fd: int | None = None
        self._lock = threading.Lock()

    def probe(self) -> StorageAvailability:
        if not self.path.is_file():
            return StorageAvailability(self.name, False, False, True, f"data file does not exist: {self.path}")
        return StorageAvailability(self.name, True, False, True, "portable buffered positioned reads")

    def _descriptor(self) -> int:
        # One descriptor per backend, opened lazily under a lock so concurrent
        # I/O workers never race to open duplicates.
        with self._lock:
            if self._fd is None:
                self._fd = os.open(self.path, os.O_RDONLY | getattr(os, "O_BINARY", 0))
            return self._fd

    def allocate_buffer(
        self,
        size: int,
        *,
        pinned: bool = False,
        device: torch.device | None = None,
    ) -> torch.Tensor:
        del device
        return host_buffer(size, pinned)

    def read_into(self, entry: BlockEntry, destination: torch.Tensor) -> None:
        if destination.device.type != "cpu":
            raise ValueError("buffered backend requires a CPU destination tensor")
        if destination.dtype != torch.uint8 or destination.numel() < entry.length:
            raise ValueError("destination must be a sufficiently large uint8 tensor")
        view = memoryview(destination[: entry.length].numpy())
        fd = self._descriptor()
        got = 0
        while got < entry.length:
            n = os.preadv(fd, [view[got:]], entry.offset + got)
            if n <= 0:
                break
            got += n
        if got != entry.length:
            raise EOFError(
                f"short read for layer={entry.layer}, block={entry.block}: "
                f"expected {entry.length}, got {got}"
            )

    def close(self) -> None:
        with self._lock:
            if self._fd is not None:
                os.close(self._fd)
                self._fd = None
