"""Positioned reads of the data file shared by the buffered and O_DIRECT
backends (the reference keeps one class per backend,
src/kvssd/storage/buffered.py:13-82 and src/kvssd/storage/direct.py:24-94).

One descriptor per backend, opened on first use under a lock (the loader's
I/O threads share it; ``preadv`` carries its own offset, so reads need no
lock).  A read fills the destination completely or raises EOFError: short
reads, which the kernel may return for large requests, are continued.
"""

from __future__ import annotations

import mmap
import os
import threading
from pathlib import Path

import torch

from ..format import ALIGNMENT, BlockEntry


def page_aligned_buffer(size: int) -> torch.Tensor:
    """``size`` bytes of anonymous memory as a CPU uint8 tensor.  mmap returns
    whole pages, so the address is page-aligned (a multiple of ALIGNMENT) by
    construction; the tensor keeps the mapping alive."""
    region = mmap.mmap(-1, max(size, 1), flags=mmap.MAP_PRIVATE | mmap.MAP_ANONYMOUS)
    buf = torch.frombuffer(region, dtype=torch.uint8)[:size]
    assert buf.data_ptr() % ALIGNMENT == 0
    return buf


class PositionedFile:
    """The data file read at explicit offsets through one lazily opened descriptor."""

    def __init__(self, path: str | Path, extra_flags: int = 0):
        self.path = Path(path)
        self._flags = os.O_RDONLY | getattr(os, "O_BINARY", 0) | extra_flags
        self._fd: int | None = None
        self._open_lock = threading.Lock()

    def descriptor(self) -> int:
        with self._open_lock:
            if self._fd is None:
                self._fd = os.open(self.path, self._flags)
            return self._fd

    def read_exact(self, offset: int, view: memoryview) -> int:
        """Bytes read into ``view`` from ``offset`` (len(view) unless the file ends)."""
        fd = self.descriptor()
        done = 0
        while done < len(view):
            n = os.preadv(fd, [view[done:]], offset + done)
            if n <= 0:
                break
            done += n
        return done

    def close(self) -> None:
        with self._open_lock:
            fd, self._fd = self._fd, None
        if fd is not None:
            os.close(fd)


def destination_view(destination: torch.Tensor, entry: BlockEntry) -> memoryview:
    return memoryview(destination[: entry.length].numpy())
