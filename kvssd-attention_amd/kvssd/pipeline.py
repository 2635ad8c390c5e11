"""Selection, SSD prefetch, pinned staging and fused decode on one GPU.

Reference: src/kvssd/pipeline.py:19-196.  The same public surface
(``KVSSDPipeline(store, device, io_depth, stage_blocks, require_cuda_kernel,
attention_backend)``, ``decode(query, layer, selector)``, context manager),
re-planned for MI355X:

* Staging uses a small ring of page-locked host slots, each laid out as the
  five PackedBatch arrays back to back, with a matching device slot.  A chunk
  is coalesced into its host slot with one ``torch.stack(out=...)`` per array
  and crosses PCIe with ``hipMemcpyAsync`` (libkvssd_hip) on the transfer
  stream: one copy for a full chunk instead of one ``.to()`` per tensor, and no
  page-locked allocation per chunk (the reference pins fresh tensors for every
  chunk, pipeline.py:98-109).
* HIP events order the streams: the compute stream waits for a slot's copy;
  the transfer stream waits for the kernel that last read the slot's device
  memory before overwriting it; the host waits for a slot's previous copy only
  before refilling that host slot.
* Each chunk's (O, LSE) folds into a running accumulator with one HIP merge
  kernel (the reference issues about six torch launches, pipeline.py:147-153).
* ``load_resident`` keeps whole layers in HBM (288 GB per MI355X); ``decode``
  of a resident layer turns the selection into a device block table and runs a
  single fused call with no SSD or PCIe traffic.
"""

from __future__ import annotations

import ctypes
import math
from collections.abc import Iterator, Sequence
from dataclasses import dataclass

import torch

from . import _native
from .attention import merge_attention_chunks, packed_attention, resolve_required
from .backends import AttentionBackend, PackedBatch
from .format import CacheSpec, PackedKVBlock
from .loader import AsyncBlockLoader
from .selectors import AllBlocks, BlockSelector
from .store import KVCacheStore

_STAGING_SLOTS = 3
_ALIGN = 256


def _aligned(n: int) -> int:
    return -(-n // _ALIGN) * _ALIGN


@dataclass
class _Layout:
    """Byte offsets of the five PackedBatch arrays inside one staging slot."""

    capacity: int
    packed: int  # bytes per block of one packed array
    scales: int  # bytes per block of one scale array
    off_kp: int
    off_vp: int
    off_ks: int
    off_vs: int
    off_valid: int
    total: int

    @classmethod
    def for_spec(cls, spec: CacheSpec, capacity: int) -> "_Layout":
        packed = spec.block_tokens * spec.kv_heads * spec.packed_dim
        scales = spec.block_tokens * spec.kv_heads * (spec.head_dim // spec.group_size) * 2
        off_kp = 0
        off_vp = off_kp + _aligned(capacity * packed)
        off_ks = off_vp + _aligned(capacity * packed)
        off_vs = off_ks + _aligned(capacity * scales)
        off_valid = off_vs + _aligned(capacity * scales)
        total = off_valid + _aligned(capacity * 4)
        return cls(capacity, packed, scales, off_kp, off_vp, off_ks, off_vs, off_valid, total)

    def views(self, buf: torch.Tensor, spec: CacheSpec, n: int) -> tuple[torch.Tensor, ...]:
        groups = spec.head_dim // spec.group_size
        pshape = (n, spec.block_tokens, spec.kv_heads, spec.packed_dim)
        sshape = (n, spec.block_tokens, spec.kv_heads, groups)
        kp = buf[self.off_kp : self.off_kp + n * self.packed].view(pshape)
        vp = buf[self.off_vp : self.off_vp + n * self.packed].view(pshape)
        ks = buf[self.off_ks : self.off_ks + n * self.scales].view(torch.float16).view(sshape)
        vs = buf[self.off_vs : self.off_vs + n * self.scales].view(torch.float16).view(sshape)
        valid = buf[self.off_valid : self.off_valid + 4 * n].view(torch.int32)
        return kp, vp, ks, vs, valid

    def spans(self, n: int) -> list[tuple[int, int]]:
        """(offset, bytes) ranges holding a chunk of n blocks; one range when full."""
        if n == self.capacity:
            return [(0, self.off_valid + 4 * n)]
        return [
            (self.off_kp, n * self.packed),
            (self.off_vp, n * self.packed),
            (self.off_ks, n * self.scales),
            (self.off_vs, n * self.scales),
            (self.off_valid, 4 * n),
        ]


class _Slot:
    def __init__(self, layout: _Layout, device: torch.device):
        self.host = torch.empty(layout.total, dtype=torch.uint8, pin_memory=True)
        self.dev = torch.empty(layout.total, dtype=torch.uint8, device=device)
        self.copied: torch.cuda.Event | None = None  # H2D from this slot finished
        self.consumed: torch.cuda.Event | None = None  # kernel reading self.dev finished


@dataclass
class _Resident:
    batch: PackedBatch
    row_of: dict[int, int]


class KVSSDPipeline:
    """End-to-end selection, SSD prefetch, pinned staging, and packed attention pipeline."""

    def __init__(
        self,
        store: KVCacheStore,
        device: str | torch.device = "cuda",
        io_depth: int = 2,
        stage_blocks: int = 4,
        require_cuda_kernel: bool = False,
        attention_backend: str | AttentionBackend | None = None,
    ):
        self.store = store
        self.device = torch.device(device)
        if self.device.type == "cuda" and not torch.cuda.is_available():
            raise RuntimeError("CUDA device requested but CUDA is unavailable")
        if stage_blocks < 1:
            raise ValueError("stage_blocks must be positive")
        self.loader = AsyncBlockLoader(store, depth=io_depth, pinned=self.device.type == "cuda", device=self.device)
        self.stage_blocks = stage_blocks
        self.require_cuda_kernel = require_cuda_kernel
        self.attention_backend = resolve_required(require_cuda_kernel, attention_backend, self.device)
        gpu = self.device.type == "cuda"
        self.transfer_stream = torch.cuda.Stream(device=self.device) if gpu else None
        self.compute_stream = torch.cuda.Stream(device=self.device) if gpu else None
        self._layout: _Layout | None = None
        self._slots: list[_Slot] = []
        self._resident: dict[int, _Resident] = {}

    # ------------------------------------------------------------ helpers ---
    @staticmethod
    def _chunks(source: Iterator[PackedKVBlock], size: int) -> Iterator[list[PackedKVBlock]]:
        chunk: list[PackedKVBlock] = []
        for block in source:
            chunk.append(block)
            if len(chunk) == size:
                yield chunk
                chunk = []
        if chunk:
            yield chunk

    def _ensure_slots(self) -> None:
        if self._slots:
            return
        self._layout = _Layout.for_spec(self.store.spec, self.stage_blocks)
        self._slots = [_Slot(self._layout, self.device) for _ in range(_STAGING_SLOTS)]

    def _stage(self, blocks: Sequence[PackedKVBlock], slot: _Slot) -> tuple[tuple[torch.Tensor, ...], torch.cuda.Event]:
        """Coalesce a chunk into a pinned slot and enqueue its H2D copy on the transfer stream."""
        assert self.transfer_stream is not None and self._layout is not None
        spec, layout, n = self.store.spec, self._layout, len(blocks)
        if slot.copied is not None:
            slot.copied.synchronize()  # the host slot is still being read by a previous copy
        kp, vp, ks, vs, valid = layout.views(slot.host, spec, n)
        torch.stack([b.key.packed for b in blocks], out=kp)
        torch.stack([b.value.packed for b in blocks], out=vp)
        torch.stack([b.key.scales for b in blocks], out=ks)
        torch.stack([b.value.scales for b in blocks], out=vs)
        valid.copy_(torch.tensor([b.valid_tokens for b in blocks], dtype=torch.int32))
        lib = _native.load()
        stream = _native.stream_handle(self.transfer_stream)
        if slot.consumed is not None:
            self.transfer_stream.wait_event(slot.consumed)
        host, dev = slot.host.data_ptr(), slot.dev.data_ptr()
        for off, nbytes in layout.spans(n):
            rc = lib.kvssd_hip_memcpy_h2d_async(ctypes.c_void_p(dev + off), ctypes.c_void_p(host + off), nbytes, stream)
            _native.check(rc, "kvssd_hip_memcpy_h2d_async")
        copied = torch.cuda.Event()
        copied.record(self.transfer_stream)
        slot.copied = copied
        return layout.views(slot.dev, spec, n), copied

    def _merge(self, acc: tuple[torch.Tensor, torch.Tensor] | None, out: torch.Tensor, lse: torch.Tensor):
        if acc is None:
            return out, lse
        merge = getattr(self.attention_backend, "merge_chunks", None)
        if merge is not None:
            merge(acc[0], acc[1], out, lse)
            return acc
        return merge_attention_chunks(acc[0], acc[1], out, lse)

    # ---------------------------------------------------------- streamed ---
    def _decode_streamed(self, query: torch.Tensor, layer: int, selected: list[int]) -> torch.Tensor:
        assert self.compute_stream is not None and self.transfer_stream is not None
        self._ensure_slots()
        chunks = self._chunks(self.loader.iter_blocks(layer, selected), self.stage_blocks)
        first = next(chunks, None)
        if first is None:
            raise ValueError("selector returned no blocks")
        spec = self.store.spec
        scale = 1.0 / math.sqrt(query.shape[-1])
        caller = torch.cuda.current_stream(self.device)
        self.compute_stream.wait_stream(caller)
        query.record_stream(self.compute_stream)
        acc: tuple[torch.Tensor, torch.Tensor] | None = None
        index = 0
        current = self._stage(first, self._slots[0])
        while current is not None:
            slot = self._slots[index % len(self._slots)]
            tensors, ready = current
            with torch.cuda.stream(self.compute_stream):
                self.compute_stream.wait_event(ready)
                out, lse = self.attention_backend.run(query, PackedBatch(*tensors, spec.bits, spec.group_size), scale)
                acc = self._merge(acc, out, lse)
                consumed = torch.cuda.Event()
                consumed.record(self.compute_stream)
                slot.consumed = consumed
            # read + stage the next chunk while the kernel runs
            nxt = next(chunks, None)
            index += 1
            current = None if nxt is None else self._stage(nxt, self._slots[index % len(self._slots)])
        assert acc is not None
        done = torch.cuda.Event()
        done.record(self.compute_stream)
        caller.wait_event(done)
        acc[0].record_stream(caller)
        return acc[0].to(query.dtype)

    # ---------------------------------------------------------- resident ---
    def load_resident(self, layers: Sequence[int] | None = None) -> None:
        """Copy whole layers into device memory; later decodes of them read HBM only."""
        if self.device.type != "cuda":
            raise RuntimeError("resident layers need a GPU device")
        spec = self.store.spec
        for layer in layers if layers is not None else range(spec.layers):
            ids = self.store.blocks_for_layer(layer)
            if not ids:
                raise ValueError(f"layer {layer} has no blocks")
            blocks = list(self.loader.iter_blocks(layer, ids))
            kp = torch.stack([b.key.packed for b in blocks]).to(self.device)
            vp = torch.stack([b.value.packed for b in blocks]).to(self.device)
            ks = torch.stack([b.key.scales for b in blocks]).to(self.device)
            vs = torch.stack([b.value.scales for b in blocks]).to(self.device)
            valid = torch.tensor([b.valid_tokens for b in blocks], dtype=torch.int32, device=self.device)
            batch = PackedBatch(kp, vp, ks, vs, valid, spec.bits, spec.group_size)
            self._resident[layer] = _Resident(batch, {bid: row for row, bid in enumerate(ids)})

    def release_resident(self, layers: Sequence[int] | None = None) -> None:
        for layer in list(self._resident) if layers is None else layers:
            self._resident.pop(layer, None)

    def _decode_resident(self, query: torch.Tensor, layer: int, selected: list[int]) -> torch.Tensor:
        res = self._resident[layer]
        rows = [res.row_of[b] for b in selected]
        scale = 1.0 / math.sqrt(query.shape[-1])
        run = self.attention_backend.run
        if getattr(self.attention_backend, "name", None) == "hip":
            out, _ = run(query, res.batch, scale, block_table=rows)
        else:
            idx = torch.tensor(rows, dtype=torch.long, device=self.device)
            b = res.batch
            sub = PackedBatch(
                b.packed_k[idx], b.packed_v[idx], b.scales_k[idx], b.scales_v[idx], b.valid_tokens[idx], b.bits, b.group_size
            )
            out, _ = run(query, sub, scale)
        return out.to(query.dtype)

    # ------------------------------------------------------------ public ---
    def decode(
        self,
        query: torch.Tensor,
        layer: int,
        selector: BlockSelector | None = None,
    ) -> torch.Tensor:
        selector = selector or AllBlocks()
        selected = selector.select(self.store.blocks_for_layer(layer))
        if not selected:
            raise ValueError("selector returned no blocks")
        query = query.to(self.device)
        if layer in self._resident:
            return self._decode_resident(query, layer, selected)
        if self.device.type == "cuda" and self.attention_backend.probe(self.device).accelerated:
            return self._decode_streamed(query, layer, selected)
        blocks = list(self.loader.iter_blocks(layer, selected))
        return packed_attention(
            query,
            blocks,
            sm_scale=1.0 / math.sqrt(query.shape[-1]),
            require_cuda_kernel=self.require_cuda_kernel,
            attention_backend=self.attention_backend,
        )

    def close(self) -> None:
        self.loader.close()
        self._resident.clear()

    def __enter__(self) -> "KVSSDPipeline":
        return self

    def __exit__(self, *_: object) -> None:
        self.close()
