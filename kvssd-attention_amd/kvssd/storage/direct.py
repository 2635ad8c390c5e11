"""Linux O_DIRECT reads into 4 KiB-aligned host buffers
(reference: src/kvssd/storage/direct.py:14-94)."""

from __future__ import annotations

import os
import sys
import threading
from pathlib import Path

import torch

from ..format import ALIGNMENT, BlockEntry
from .base import StorageAvailability


def aligned_host_buffer(size: int, *, pinned: bool = False) -> torch.Tensor:
    """A CPU uint8 view of ``size`` bytes whose address is ALIGNMENT-aligned."""
    owner = torch.empty(size + ALIGNMENT - 1, dtype=torch.uint8, pin_memory=pinned and torch.cuda.is_available())
    shift = (-owner.data_ptr()) % ALIGNMENT
    return owner[shift : shift + size]


class DirectIOStorageBackend:
    """Linux O_DIRECT positioned reads; offsets, lengths and addresses are checked."""

    name = "direct"

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._fd: int | None = None
        self._lock = threading.Lock()

    def probe(self) -> StorageAvailability:
        if sys.platform != "linux" or not hasattr(os, "O_DIRECT"):
            return StorageAvailability(self.name, False, True, True, "O_DIRECT requires Linux")
        if not self.path.is_file():
            return StorageAvailability(self.name, False, True, True, f"data file does not exist: {self.path}")
        try:
            os.close(os.open(self.path, os.O_RDONLY | os.O_DIRECT))
        except OSError as exc:
            return StorageAvailability(self.name, False, True, True, f"O_DIRECT open failed: {exc}")
        return StorageAvailability(self.name, True, True, True, "Linux O_DIRECT positioned reads")

    def _descriptor(self) -> int:
        with self._lock:
            if self._fd is None:
                self._fd = os.open(self.path, os.O_RDONLY | os.O_DIRECT)
            return self._fd

    def allocate_buffer(
        self,
        size: int,
        *,
        pinned: bool = False,
        device: torch.device | None = None,
    ) -> torch.Tensor:
        # ROCm page-locked memory is not a valid O_DIRECT target (preadv fails
        # with EFAULT), so direct-read buffers are always pageable.
        del device, pinned
        return aligned_host_buffer(size, pinned=False)

    def read_into(self, entry: BlockEntry, destination: torch.Tensor) -> None:
        if destination.device.type != "cpu" or destination.dtype != torch.uint8:
            raise ValueError("direct backend requires a CPU uint8 destination")
        if destination.numel() < entry.length:
            raise ValueError("destination is smaller than the requested record")
        if entry.offset % ALIGNMENT or entry.length % ALIGNMENT:
            raise ValueError(
                f"unaligned direct read for layer={entry.layer}, block={entry.block}: "
                f"offset={entry.offset}, length={entry.length}, alignment={ALIGNMENT}"
            )
        if destination.data_ptr() % ALIGNMENT:
            raise ValueError(
                f"direct destination address must be {ALIGNMENT}-byte aligned; "
                f"got address=0x{destination.data_ptr():x}"
            )
        got = os.preadv(self._descriptor(), [memoryview(destination[: entry.length].numpy())], entry.offset)
        if got != entry.length:
            raise EOFError(
                f"short direct read for layer={entry.layer}, block={entry.block}: "
                f"offset={entry.offset}, expected={entry.length}, got={got}"
            )

    def close(self) -> None:
        with self._lock:
            if self._fd is not None:
                os.close(self._fd)
                self._fd = None
