"""Bounded prefetcher of KV records (reference: src/kvssd/loader.py:22-137).

Reads stay on the host (O_DIRECT/preadv through the storage backend) in a
small thread pool; ``depth`` reusable slots bound the bytes in flight.  Each
yielded block owns copies of its four payload tensors, so recycling a slot can
never corrupt a block a consumer still holds.

``read_records`` is the record-native form used by the GPU pipeline: raw
records land in the rows of a caller's buffer (the pipeline's page-locked
staging slot) with no parsing, CRC or copies on the host; the GPU gather
verifies them.

The slots are pageable host memory even when ``pinned=True`` is passed: on
ROCm, page-locked memory from the HIP runtime is not a valid O_DIRECT target
(``preadv`` fails with EFAULT), and the slots are only bounce buffers anyway;
the pipeline's page-locked staging ring is what crosses PCIe.
"""

from __future__ import annotations

from collections import deque
from collections.abc import Callable, Sequence
from concurrent.futures import Future, ThreadPoolExecutor
from dataclasses import dataclass
from queue import Queue
from typing import Iterator

import torch

from .format import BlockEntry, PackedKVBlock, decode_record
from .quant import QuantizedTensor
from .store import KVCacheStore


@dataclass
class _Slot:
    raw: torch.Tensor
    future: Future[PackedKVBlock] | None = None


def _detach(block: PackedKVBlock) -> PackedKVBlock:
    def own(q: QuantizedTensor) -> QuantizedTensor:
        return QuantizedTensor(q.packed.clone(), q.scales.clone(), q.original_shape, q.bits, q.group_size)

    return PackedKVBlock(block.layer, block.block, block.valid_tokens, own(block.key), own(block.value))


class AsyncBlockLoader:
    """Bounded pinned-memory prefetcher; slots provide backpressure by construction."""

    def __init__(
        self,
        store: KVCacheStore,
        depth: int = 2,
        pinned: bool = True,
        device: torch.device | None = None,
    ):
        if depth < 1:
            raise ValueError("depth must be positive")
        self.store = store
        self.device = device
        self.executor = ThreadPoolExecutor(max_workers=depth, thread_name_prefix="kvssd-io")
        self.free: Queue[_Slot] = Queue()
        del pinned  # see the module docstring: slots stay pageable
        for _ in range(depth):
            raw = store.storage_backend.allocate_buffer(store.spec.record_bytes, pinned=False, device=device)
            self.free.put(_Slot(raw))
        # O_DIRECT needs its own aligned pageable target; other backends read
        # straight into the caller's rows
        self._bounce = bool(store.storage_backend.probe().direct)

    def iter_blocks(self, layer: int, block_ids: list[int]) -> Iterator[PackedKVBlock]:
        pending: deque[tuple[_Slot, BlockEntry]] = deque()
        todo = iter(block_ids)

        def work(entry: BlockEntry, raw: torch.Tensor) -> PackedKVBlock:
            # read, verify the CRC and copy the payloads out, all on the I/O
            # thread; zlib and preadv release the GIL
            self.store.read_into(entry, raw)
            return _detach(decode_record(raw, self.store.spec))

        def submit(block_id: int) -> None:
            slot = self.free.get()
            entry = self.store.entry(layer, block_id)
            slot.future = self.executor.submit(work, entry, slot.raw)
            pending.append((slot, entry))

        for _ in range(min(self.free.qsize(), len(block_ids))):
            submit(next(todo))
        while pending:
            slot, entry = pending.popleft()
            assert slot.future is not None
            block = slot.future.result()
            nxt = next(todo, None)
            self.free.put(slot)
            if nxt is not None:
                submit(nxt)
            yield block

    def read_records(self, layer: int, block_ids: Sequence[int], destination: torch.Tensor) -> None:
        """Raw records of ``block_ids`` into rows 0..n-1 of ``destination``
        (a contiguous CPU uint8 tensor [>= n, record_bytes]), read on the I/O
        threads.  No header or CRC check happens here."""
        self.read_records_async(layer, block_ids, destination)()

    def read_records_async(
        self, layer: int, block_ids: Sequence[int], destination: torch.Tensor
    ) -> Callable[[], None]:
        """As read_records, returning as soon as the reads are queued; the
        returned callable waits for all of them and raises the first error."""
        rb = self.store.spec.record_bytes
        if (
            destination.device.type != "cpu"
            or destination.dtype != torch.uint8
            or destination.dim() != 2
            or destination.shape[1] != rb
            or destination.shape[0] < len(block_ids)
            or not destination.is_contiguous()
        ):
            raise ValueError(f"destination must be a contiguous CPU uint8 tensor [>= {len(block_ids)}, {rb}]")
        entries = [self.store.entry(layer, b) for b in block_ids]
        for entry in entries:
            if entry.length != rb:
                raise ValueError("record layout does not match manifest")

        def work(entry: BlockEntry, row: torch.Tensor) -> None:
            if not self._bounce:
                self.store.read_into(entry, row)
                return
            slot = self.free.get()
            try:
                self.store.read_into(entry, slot.raw)
                row.copy_(slot.raw[:rb])
            finally:
                self.free.put(slot)

        futures = [self.executor.submit(work, e, destination[i]) for i, e in enumerate(entries)]

        def wait() -> None:
            # every read finishes before the first error is raised, so no
            # worker still writes into the destination afterwards
            errors = [f.exception() for f in futures]
            for err in errors:
                if err is not None:
                    raise err

        return wait

    def close(self) -> None:
        self.executor.shutdown(wait=True, cancel_futures=False)

    def __enter__(self) -> "AsyncBlockLoader":
        return self

    def __exit__(self, *_: object) -> None:
        self.close()
