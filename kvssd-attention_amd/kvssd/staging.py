"""Record-native staging ring and chunk loop of the streamed GPU decode.

Reference: KVSSDPipeline._chunks / _stage / _decode_cuda_streamed
(src/kvssd/pipeline.py:56-165).  The reference parses every record on the host
(CRC, four payload clones, src/kvssd/loader.py:73-91), stacks a chunk into
freshly pinned tensors and copies each tensor H2D (pipeline.py:98-114).  Here a
chunk stays in the on-disk record form end to end:

* the raw records of a chunk sit back to back in page-locked host memory -- a
  staging slot the loader reads into, or a whole layer kept in host memory --
  and cross PCIe with one ``hipMemcpyAsync`` per run of consecutive records;
  successive chunks alternate between two transfer streams, which keeps two
  copy engines busy (56 GB/s host-to-device on MI355X against 53.5 GB/s from
  one);
* on the compute stream ``kvssd_hip_gather_records`` checks each record's
  header, layout and payload CRC-32 and writes the slot's PackedBatch arrays;
  the fused decode reads them and one merge kernel folds the chunk's (O, LSE)
  into the running result;
* HIP events order the two streams: the compute stream waits for a slot's
  copy; before a slot is refilled the host waits for the kernels that last
  read its device memory (and, for a staging slot, for its previous copy).
  The transfer stream itself never waits on a compute-stream event: on
  MI355X a copy-engine queue that waits on a kernel queue's event loses tens
  of microseconds per chunk, while the host-side wait costs nothing when the
  ring is deep enough that it rarely blocks.

Record statuses of the whole decode collect in one device vector, read back
once at the end: a bad header or layout raises ValueError and a CRC mismatch
IOError, with decode_record's messages (src/kvssd/format.py:140-152).
"""

from __future__ import annotations

import ctypes
import time
from collections.abc import Callable, Sequence
from dataclasses import dataclass

import torch

from . import _native
from .attention import merge_attention_chunks
from .backends import AttentionBackend, PackedBatch
from .backends.hip import HipAttentionBackend
from .format import CacheSpec
from .records_hip import gather_records, raise_for_status

SLOTS = 3
_ALIGN = 256

# (host address, byte offset into the slot's device records, bytes)
Span = tuple[int, int, int]


def _aligned(n: int) -> int:
    return -(-n // _ALIGN) * _ALIGN


@dataclass
class BatchLayout:
    """Byte offsets of the five PackedBatch arrays inside one device buffer."""

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
    def for_spec(cls, spec: CacheSpec, capacity: int) -> "BatchLayout":
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


class Slot:
    """One staging slot: ``capacity`` raw records in page-locked host memory,
    the same bytes on the device, and the PackedBatch arrays gathered from them."""

    def __init__(self, spec: CacheSpec, layout: BatchLayout, device: torch.device):
        nbytes = layout.capacity * spec.record_bytes
        self.host = torch.empty((layout.capacity, spec.record_bytes), dtype=torch.uint8, pin_memory=True)
        self.raw = torch.empty(nbytes, dtype=torch.uint8, device=device)
        self.batch = torch.empty(layout.total, dtype=torch.uint8, device=device)
        self.copied: torch.cuda.Event | None = None  # H2D into self.raw finished
        self.consumed: torch.cuda.Event | None = None  # kernels reading self.raw / self.batch finished
        self._events = (torch.cuda.Event(), torch.cuda.Event())

    def copied_event(self) -> torch.cuda.Event:
        """This slot's copy event, re-recorded for every chunk."""
        self.copied = self._events[0]
        return self.copied

    def consumed_event(self) -> torch.cuda.Event:
        self.consumed = self._events[1]
        return self.consumed

    def host_ready(self) -> None:
        """Block until no copy still reads this slot's host memory."""
        if self.copied is not None:
            self.copied.synchronize()


@dataclass
class HostRecords:
    """Raw records of one layer kept in page-locked host memory: ``records``
    uint8 [n, record_bytes], row i holding block ``block_ids[i]``."""

    records: torch.Tensor
    block_ids: list[int]

    def __post_init__(self) -> None:
        self.row_of = {b: i for i, b in enumerate(self.block_ids)}

    def spans(self, ids: Sequence[int], record_bytes: int) -> list[Span]:
        """One span per run of consecutive rows, in the order of ``ids``."""
        base = self.records.data_ptr()
        out: list[Span] = []
        rows = [self.row_of[b] for b in ids]
        start = 0
        for j in range(1, len(rows) + 1):
            if j == len(rows) or rows[j] != rows[j - 1] + 1:
                out.append((base + rows[start] * record_bytes, start * record_bytes, (j - start) * record_bytes))
                start = j
        return out


# fill(ids, slot) puts the raw records of ``ids`` where the returned spans point
Fill = Callable[[Sequence[int], Slot], list[Span]]


class ReadFill:
    """Chunks read from storage into a slot's page-locked host memory, one
    chunk ahead of the one being staged: ``prefetch`` queues the reads of a
    later chunk (once the slot's previous copy out of that memory is done) and
    the fill of that chunk waits for them, so the loader's threads read chunk
    i + 2 while chunk i + 1 crosses PCIe and chunk i is decoded."""

    def __init__(self, record_bytes: int, read: Callable[[Sequence[int], torch.Tensor], Callable[[], None]]):
        self.record_bytes = record_bytes
        self.read = read
        self.pending: dict[int, tuple[tuple[int, ...], Callable[[], None]]] = {}

    def prefetch(self, ids: Sequence[int], slot: Slot) -> None:
        self.drain(slot)
        slot.host_ready()
        self.pending[id(slot)] = (tuple(ids), self.read(ids, slot.host))

    def drain(self, slot: Slot) -> None:
        got = self.pending.pop(id(slot), None)
        if got is not None:
            got[1]()

    def drain_all(self) -> None:
        """Wait for every queued read (a run that stops early leaves none behind)."""
        pending, self.pending = self.pending, {}
        errors = []
        for _, wait in pending.values():
            try:
                wait()
            except Exception as exc:  # reported only if nothing else was raised
                errors.append(exc)
        if errors:
            raise errors[0]

    def __call__(self, ids: Sequence[int], slot: Slot) -> list[Span]:
        got = self.pending.pop(id(slot), None)
        if got is not None and got[0] == tuple(ids):
            got[1]()
        else:
            if got is not None:
                got[1]()
            slot.host_ready()
            self.read(ids, slot.host)()
        return [(slot.host.data_ptr(), 0, len(ids) * self.record_bytes)]


class RecordStager:
    """Staging ring plus chunk loop: ``run`` attends over the records of
    ``block_ids`` in chunks of ``stage_blocks`` and returns (out f32, lse f32)."""

    def __init__(
        self,
        spec: CacheSpec,
        device: torch.device,
        stage_blocks: int,
        backend: AttentionBackend,
        transfer_stream: torch.cuda.Stream | Sequence[torch.cuda.Stream],
        compute_stream: torch.cuda.Stream,
        slots: int = SLOTS,
    ):
        if stage_blocks < 1:
            raise ValueError("stage_blocks must be positive")
        if slots < 2:
            raise ValueError("the staging ring needs at least two slots")
        self.spec = spec
        self.device = device
        self.stage_blocks = stage_blocks
        self.backend = backend
        if isinstance(transfer_stream, torch.cuda.Stream):
            transfer_stream = [transfer_stream]
        self.transfer_streams = list(transfer_stream)
        if not self.transfer_streams:
            raise ValueError("at least one transfer stream is required")
        self.compute_stream = compute_stream
        self.layout = BatchLayout.for_spec(spec, stage_blocks)
        self.slots = [Slot(spec, self.layout, device) for _ in range(slots)]
        self._record_layout = _native.RecordLayout(
            spec.bits, spec.block_tokens, spec.kv_heads, spec.head_dim, spec.group_size
        )
        self.last_enqueue_seconds = 0.0  # host time the last run spent issuing its chunks
        # record statuses of a run whose check is deferred: (event, host codes, layer, ids)
        self.defer_checks = False
        self._pending: tuple[torch.cuda.Event, torch.Tensor, int, list[int]] | None = None

    # ------------------------------------------------------------- fills ---
    def host_fill(self, host: HostRecords) -> Fill:
        """Chunks copied straight from a layer kept in page-locked memory."""
        rb = self.spec.record_bytes
        return lambda ids, slot: host.spans(ids, rb)

    def read_fill(self, read: Callable[[Sequence[int], torch.Tensor], Callable[[], None]]) -> "ReadFill":
        """Chunks read into the slot's host memory by ``read(ids, rows)``,
        which queues the reads and returns their waiter."""
        return ReadFill(self.spec.record_bytes, read)

    # -------------------------------------------------------------- loop ---
    def _stage(self, index: int, ids: Sequence[int], fill: Fill) -> None:
        """Enqueue the copy of chunk ``index`` into its slot."""
        slot = self.slots[index % len(self.slots)]
        transfer = self.transfer_streams[index % len(self.transfer_streams)]
        spans = fill(ids, slot)
        if slot.consumed is not None:
            slot.consumed.synchronize()  # kernels of this slot's previous chunk are done
        lib = _native.load()
        stream = _native.stream_handle(transfer)
        dev = slot.raw.data_ptr()
        for src, off, nbytes in spans:
            rc = lib.kvssd_hip_memcpy_h2d_async(ctypes.c_void_p(dev + off), ctypes.c_void_p(src), nbytes, stream)
            _native.check(rc, "kvssd_hip_memcpy_h2d_async")
        slot.copied_event().record(transfer)

    def _prefetch(self, index: int, chunks: list[list[int]], fill: Fill) -> None:
        """Queue the reads of chunk ``index`` into its slot, if the fill reads."""
        prefetch = getattr(fill, "prefetch", None)
        if prefetch is not None and index < len(chunks):
            prefetch(chunks[index], self.slots[index % len(self.slots)])

    def _merge(self, acc, out: torch.Tensor, lse: torch.Tensor):
        if acc is None:
            return out, lse
        merge = getattr(self.backend, "merge_chunks", None)
        if merge is not None:
            merge(acc[0], acc[1], out, lse)
            return acc
        return merge_attention_chunks(acc[0], acc[1], out, lse)

    def check_pending(self) -> None:
        """Raise for the records of a deferred run (blocks until it finished)."""
        pending, self._pending = self._pending, None
        if pending is not None:
            event, codes, layer, ids = pending
            event.synchronize()
            raise_for_status(codes, layer, ids)

    def run(
        self, query: torch.Tensor, sm_scale: float, layer: int, block_ids: Sequence[int], fill: Fill
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Attention over the records of ``block_ids``.  Their statuses are
        checked before the call returns (the reference's behaviour), or, with
        ``defer_checks``, at the start of the next run or in check_pending, so
        that a loop over layers never waits for the GPU."""
        self.check_pending()
        chunks = [list(block_ids[i : i + self.stage_blocks]) for i in range(0, len(block_ids), self.stage_blocks)]
        if not chunks:
            raise ValueError("selector returned no blocks")
        compute = self.compute_stream
        caller = torch.cuda.current_stream(self.device)
        compute.wait_stream(caller)
        query.record_stream(compute)
        with torch.cuda.stream(compute):
            status = torch.empty(len(block_ids), dtype=torch.int32, device=self.device)
            t0 = time.perf_counter()
            try:
                if isinstance(self.backend, HipAttentionBackend) and query.dtype in _native.QUERY_DTYPES:
                    acc = self._loop_native(query, sm_scale, chunks, fill, status)
                else:
                    acc = self._loop_generic(query, sm_scale, chunks, fill, status)
            finally:
                drain_all = getattr(fill, "drain_all", None)
                if drain_all is not None:
                    drain_all()
            self.last_enqueue_seconds = time.perf_counter() - t0
            codes = torch.empty(status.shape, dtype=status.dtype, pin_memory=True)
            codes.copy_(status, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record(compute)
        self._pending = (ready, codes, layer, list(block_ids))
        if not self.defer_checks:
            self.check_pending()
        done = torch.cuda.Event()
        done.record(compute)
        caller.wait_event(done)
        for t in acc:
            t.record_stream(caller)
        return acc

    def _loop_generic(self, query, sm_scale, chunks, fill, status):
        """Any attention backend: PackedBatch views of the gathered slot."""
        spec, sb, compute = self.spec, self.stage_blocks, self.compute_stream
        acc = None
        self._stage(0, chunks[0], fill)
        self._prefetch(1, chunks, fill)
        for i, ids in enumerate(chunks):
            slot = self.slots[i % len(self.slots)]
            n = len(ids)
            assert slot.copied is not None
            compute.wait_event(slot.copied)
            arrays = self.layout.views(slot.batch, spec, n)
            gather_records(slot.raw, spec, n, out=(*arrays, status[i * sb : i * sb + n]))
            out, lse = self.backend.run(query, PackedBatch(*arrays, spec.bits, spec.group_size), sm_scale)
            acc = self._merge(acc, out, lse)
            slot.consumed_event().record(compute)
            if i + 1 < len(chunks):
                self._stage(i + 1, chunks[i + 1], fill)
                self._prefetch(i + 2, chunks, fill)
        assert acc is not None
        return acc

    def _loop_native(self, query, sm_scale, chunks, fill, status):
        """The hip backend: every per-chunk launch goes straight to the C ABI
        with descriptors and pointers prepared once per decode, so the host
        spends a few ctypes calls per chunk and keeps ahead of the copies."""
        spec, sb, compute = self.spec, self.stage_blocks, self.compute_stream
        lib = _native.load()
        q = query.contiguous()
        # the reference's argument checks, once (every chunk has the same shape)
        PackedBatch(*self.layout.views(self.slots[0].batch, spec, 1), spec.bits, spec.group_size).validate(q)
        qh, dim = q.shape
        descs: dict[int, _native.DecodeDesc] = {}
        need = 1
        for n in {len(c) for c in chunks}:
            d = _native.DecodeDesc(
                query_heads=qh,
                kv_heads=spec.kv_heads,
                head_dim=dim,
                num_blocks=n,
                block_tokens=spec.block_tokens,
                bits=spec.bits,
                group_size=spec.group_size,
                query_dtype=_native.QUERY_DTYPES[q.dtype],
                num_selected=0,
                kernel=self.backend.kernel,
                sm_scale=float(sm_scale),
            )
            nbytes = ctypes.c_size_t(0)
            _native.check(lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(d), ctypes.byref(nbytes)), "workspace")
            need = max(need, int(nbytes.value))
            descs[n] = d
        work = torch.empty(need, dtype=torch.uint8, device=self.device)
        acc_out = torch.empty((qh, dim), dtype=torch.float32, device=self.device)
        acc_lse = torch.empty(qh, dtype=torch.float32, device=self.device)
        tmp_out = torch.empty_like(acc_out)
        tmp_lse = torch.empty_like(acc_lse)
        cs = _native.stream_handle(compute)
        lay = ctypes.byref(self._record_layout)
        L, rb = self.layout, spec.record_bytes
        qp, wp = q.data_ptr(), work.data_ptr()
        sp = status.data_ptr()
        self._stage(0, chunks[0], fill)
        self._prefetch(1, chunks, fill)
        for i, ids in enumerate(chunks):
            slot = self.slots[i % len(self.slots)]
            n = len(ids)
            assert slot.copied is not None
            compute.wait_event(slot.copied)
            b = slot.batch.data_ptr()
            kp, vp, ks, vs, va = b + L.off_kp, b + L.off_vp, b + L.off_ks, b + L.off_vs, b + L.off_valid
            rc = lib.kvssd_hip_gather_records(lay, slot.raw.data_ptr(), rb, n, 1, kp, vp, ks, vs, va, sp + 4 * i * sb, cs)
            _native.check(rc, "kvssd_hip_gather_records")
            o, l = (acc_out, acc_lse) if i == 0 else (tmp_out, tmp_lse)
            rc = lib.kvssd_hip_fused_decode(
                ctypes.byref(descs[n]), qp, kp, vp, ks, vs, va, None, o.data_ptr(), l.data_ptr(), wp, need, cs
            )
            _native.check(rc, "kvssd_hip_fused_decode")
            if i:
                rc = lib.kvssd_hip_merge_chunks(
                    qh, dim, acc_out.data_ptr(), acc_lse.data_ptr(), tmp_out.data_ptr(), tmp_lse.data_ptr(), cs
                )
                _native.check(rc, "kvssd_hip_merge_chunks")
            slot.consumed_event().record(compute)
            if i + 1 < len(chunks):
                self._stage(i + 1, chunks[i + 1], fill)
                self._prefetch(i + 2, chunks, fill)
        return acc_out, acc_lse
