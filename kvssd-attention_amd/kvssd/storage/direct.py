"""O_DIRECT positioned reads that bypass the page cache (the reference's
``direct`` backend, src/kvssd/storage/direct.py:24-94).

O_DIRECT needs the file offset, the length and the destination address to be
multiples of the block size (ALIGNMENT, 4 KiB); each is checked before the
read with the reference's messages.  Buffers come from anonymous mmap (page
aligned by construction).  They are pageable even when ``pinned=True`` is
asked for: page-locked memory from the ROCm runtime is not a valid O_DIRECT
target (the read fails with EFAULT), so the loader reads into these buffers
and copies into its page-locked staging rows.
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import torch

from ..format import ALIGNMENT, BlockEntry
from .base import StorageAvailability
from .posix import PositionedFile, destination_view, page_aligned_buffer


class DirectIOStorageBackend(PositionedFile):
    name = "direct"

    def __init__(self, path: str | Path):
        super().__init__(path, getattr(os, "O_DIRECT", 0))

    def probe(self) -> StorageAvailability:
        def state(ok: bool, why: str) -> StorageAvailability:
            return StorageAvailability(self.name, ok, True, True, why)

        if sys.platform != "linux" or not hasattr(os, "O_DIRECT"):
            return state(False, "O_DIRECT requires Linux")
        if not self.path.is_file():
            return state(False, f"data file does not exist: {self.path}")
        try:
            fd = os.open(self.path, os.O_RDONLY | os.O_DIRECT)
        except OSError as exc:
            return state(False, f"O_DIRECT open failed: {exc}")
        os.close(fd)
        return state(True, "Linux O_DIRECT positioned reads")

    def allocate_buffer(self, size: int, *, pinned: bool = False, device: torch.device | None = None) -> torch.Tensor:
        return page_aligned_buffer(size)

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
                f"direct destination address must be {ALIGNMENT}-byte aligned; got address=0x{destination.data_ptr():x}"
            )
        got = self.read_exact(entry.offset, destination_view(destination, entry))
        if got != entry.length:
            raise EOFError(
                f"short direct read for layer={entry.layer}, block={entry.block}: "
                f"offset={entry.offset}, expected={entry.length}, got={got}"
            )
