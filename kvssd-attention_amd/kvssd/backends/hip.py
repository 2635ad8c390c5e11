"""``hip`` attention backend: the fused INT2/INT4 decode kernels on gfx950.

Takes over the role of the reference's CudaExtensionBackend
(src/kvssd/backends/cuda.py:17-48), calling libkvssd_hip.so through its C ABI
(include/kvssd_hip.h) instead of the torch extension ``kvssd._C``.

* ``probe`` reports available only on a ROCm build of torch with a visible
  gfx950 device and the library loaded (checked once per device).
* ``run`` validates the batch exactly like the reference, checks dtypes as
  csrc/bindings.cpp:34-36 does, allocates out / lse / workspace with torch on
  the query's device and launches on torch's current stream.  It never
  synchronises the host and never reads device tensors back (no
  ``.tolist()`` as in src/kvssd/backends/triton.py:170).
* There is no fallback: a missing library or device raises.
"""

from __future__ import annotations

import ctypes
from collections.abc import Sequence

import torch

from .. import _native
from .base import BackendAvailability, PackedBatch

_device_state: dict[int, tuple[bool, str]] = {}


# The current stream's raw handle without building a Stream object (~0.2
# against ~1.9 us per call): torch's generated bindings read it through this
# private hook; where a torch build lacks it, the public Stream path serves.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def current_stream_handle(index: int) -> int:
    if _RAW_STREAM is not None:
        return int(_RAW_STREAM(index))
    return int(torch.cuda.current_stream(index).cuda_stream)


# The current device's index; the hook torch.cuda.current_device() ends in,
# without its lazy-initialisation check (the device is initialised by the time
# a prepared decode exists).
_CURRENT_DEVICE = getattr(torch._C, "_cuda_getDevice", None) or torch.cuda.current_device


def _index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


class HipAttentionBackend:
    name = "hip"

    def __init__(self, kernel: str = "auto"):
        names = {v: k for k, v in _native.KERNEL_NAMES.items()}
        if kernel not in names:
            raise ValueError(f"unknown hip kernel '{kernel}'; choose one of: {', '.join(names)}")
        self.kernel = names[kernel]
        self.last_kernel: str | None = None
        self._plans: dict[tuple[int, ...], tuple[int, int]] = {}

    # ------------------------------------------------------------ probe ---
    def probe(self, device: torch.device) -> BackendAvailability:
        device = torch.device(device)

        def no(reason: str) -> BackendAvailability:
            return BackendAvailability(self.name, False, True, False, reason, device.type)

        if device.type != "cuda":
            return no(f"HIP backend requires a ROCm GPU device, got {device.type}")
        if torch.version.hip is None:
            return no("HIP backend requires a ROCm build of PyTorch")
        if not torch.cuda.is_available():
            return no("no ROCm GPU is visible")
        ok, why = _native.available()
        if not ok:
            return no(why)
        index = _index(device)
        if index not in _device_state:
            _device_state[index] = _native.device_ok(index)
        ok, why = _device_state[index]
        if not ok:
            return no(why)
        return BackendAvailability(self.name, True, True, False, f"fused HIP kernels on {why}", device.type)

    # -------------------------------------------------------------- run ---
    def describe(
        self, query: torch.Tensor, batch: PackedBatch, sm_scale: float, num_selected: int = 0
    ) -> _native.DecodeDesc:
        nb, bt, kvh, _ = batch.packed_k.shape
        if query.dtype not in _native.QUERY_DTYPES:
            raise ValueError(f"unsupported query dtype {query.dtype}")
        return _native.DecodeDesc(
            query_heads=query.shape[0],
            kv_heads=kvh,
            head_dim=query.shape[1],
            num_blocks=nb,
            block_tokens=bt,
            bits=batch.bits,
            group_size=batch.group_size,
            query_dtype=_native.QUERY_DTYPES[query.dtype],
            num_selected=num_selected,
            kernel=self.kernel,
            sm_scale=float(sm_scale),
        )

    def kernel_for(self, query: torch.Tensor, batch: PackedBatch, sm_scale: float = 1.0) -> str:
        """Name of the kernel ``run`` would launch for this shape ("general", "mfma" or "staged")."""
        desc = self.describe(query, batch, sm_scale)
        out = ctypes.c_int(0)
        _native.check(_native.load().kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(out)), "decode_kernel")
        return _native.KERNEL_NAMES[out.value]

    def run(
        self,
        query: torch.Tensor,
        batch: PackedBatch,
        sm_scale: float,
        block_table: torch.Tensor | Sequence[int] | None = None,
        out_dtype: torch.dtype | None = None,
    ) -> tuple[torch.Tensor, torch.Tensor]:
        """Fused decode; with ``block_table`` attend over those block ids of the batch, in order.

        ``out`` is fp32 (the reference's output) unless ``out_dtype`` is the
        query's dtype: then the merge stores it in that dtype, rounded to
        nearest even -- the values ``out.to(query.dtype)`` would give, without
        the extra cast kernel.  ``lse`` is fp32 either way."""
        return self.prepare(query, batch, sm_scale, block_table, out_dtype)(query)

    def prepare(
        self,
        query: torch.Tensor,
        batch: PackedBatch,
        sm_scale: float,
        block_table: torch.Tensor | Sequence[int] | None = None,
        out_dtype: torch.dtype | None = None,
    ) -> "PreparedDecode":
        """Every check and plan of ``run`` for this batch, selection and query
        shape, done once; calling the result with a query of that shape, dtype
        and device decodes (what a decode loop over a resident layer repeats)."""
        return PreparedDecode(self, query, batch, sm_scale, block_table, out_dtype)

    def _plan(self, lib, desc: _native.DecodeDesc) -> tuple[int, int]:
        """(workspace bytes, kernel id) of a decode shape, asked of the library once per shape."""
        key = (
            desc.query_heads, desc.kv_heads, desc.head_dim, desc.num_blocks, desc.block_tokens,
            desc.bits, desc.group_size, desc.query_dtype, desc.num_selected,
        )
        plan = self._plans.get(key)
        if plan is None:
            need = ctypes.c_size_t(0)
            _native.check(lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(need)), "workspace")
            kern = ctypes.c_int(0)
            _native.check(lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(kern)), "decode_kernel")
            plan = (int(need.value), int(kern.value))
            if len(self._plans) >= 64:
                self._plans.clear()
            self._plans[key] = plan
        return plan

    @staticmethod
    def _staged_aligned(pk, pv, sk, sv) -> bool:
        return all(t.data_ptr() % 16 == 0 for t in (pk, pv, sk, sv))

    @staticmethod
    def _mfma_aligned(bits: int, pk, pv, sk, sv) -> bool:
        need = 16 if bits == 4 else 8
        return all(t.data_ptr() % need == 0 for t in (pk, pv)) and all(t.data_ptr() % 8 == 0 for t in (sk, sv))

    @staticmethod
    def _table(block_table, num_blocks: int, device: torch.device) -> torch.Tensor:
        if isinstance(block_table, torch.Tensor):
            if block_table.device.type == "cuda":
                # validated by the caller that built it on the device; the
                # kernels also skip ids outside [0, num_blocks)
                return block_table.to(torch.int32).contiguous()
            ids = block_table.to(torch.int64).tolist()
        else:
            ids = [int(x) for x in block_table]
        if not ids:
            raise ValueError("at least one block is required")
        if min(ids) < 0 or max(ids) >= num_blocks:
            raise ValueError(f"block ids must lie in [0, {num_blocks})")
        return torch.tensor(ids, dtype=torch.int32).pin_memory().to(device, non_blocking=True)

    # ----------------------------------------------------------- merge ---
    def merge_chunks(
        self, acc_out: torch.Tensor, acc_lse: torch.Tensor, out: torch.Tensor, lse: torch.Tensor
    ) -> None:
        """In-place exact merge (acc_out, acc_lse) <- merge((acc_out, acc_lse), (out, lse))."""
        for t in (acc_out, acc_lse, out, lse):
            if t.dtype != torch.float32 or not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError("merge operands must be contiguous fp32 GPU tensors")
        rows, dim = acc_out.shape
        if out.shape != acc_out.shape or acc_lse.shape != (rows,) or lse.shape != (rows,):
            raise ValueError("merge operand shapes differ")
        stream = torch.cuda.current_stream(acc_out.device)
        rc = _native.load().kvssd_hip_merge_chunks(
            rows, dim, _ptr(acc_out), _ptr(acc_lse), _ptr(out), _ptr(lse), _native.stream_handle(stream)
        )
        _native.check(rc, "kvssd_hip_merge_chunks")


class PreparedDecode:
    """One decode shape over one packed batch with its checks, descriptor,
    device pointers, kernel choice and workspace size fixed at construction
    (the checks of HipAttentionBackend.run, csrc/bindings.cpp:34-36 and
    src/kvssd/backends/base.py:29-55).  A call takes a query of the prepared
    shape, dtype and device and returns (out, lse) like ``run``.

    The split partials go to a workspace kept per stream: calls on one stream
    are ordered, so each reuses it; calls on another stream get their own.
    The object holds references to the batch arrays (and block table), so
    the pointers it passes stay valid while it lives.

    Every call returns a fresh (out, lse) pair, as ``run`` does, but not from
    two allocations: per stream the object allocates blocks of ``_ROWS``
    outputs at once (on that stream, so torch's allocator orders their reuse
    as it would a single tensor's) and hands out the next row of the current
    block, whose views were made with the block.  A returned tensor is a
    contiguous row of its block and keeps the block's storage alive (64 rows
    of [QH, D] plus [QH]); two calls never share a row."""

    _MAX_STREAMS = 8
    _ROWS = 64

    def __init__(self, backend: HipAttentionBackend, query, batch, sm_scale, block_table, out_dtype):
        if out_dtype is not None and out_dtype not in (torch.float32, query.dtype):
            raise ValueError(f"out_dtype must be torch.float32 or the query's dtype {query.dtype}, got {out_dtype}")
        typed = out_dtype is not None and out_dtype != torch.float32
        batch.validate(query)
        if query.device.type != "cuda":
            raise ValueError(f"HIP backend requires ROCm GPU tensors, got {query.device.type}")
        if batch.packed_k.dtype != torch.uint8 or batch.packed_v.dtype != torch.uint8:
            raise ValueError("packed KV must be uint8")
        if batch.scales_k.dtype != torch.float16 or batch.scales_v.dtype != torch.float16:
            raise ValueError("scales must be float16")
        if batch.valid_tokens.dtype != torch.int32:
            raise ValueError("valid_tokens must be int32")
        if batch.scales_k.shape[:3] != batch.packed_k.shape[:3] or batch.scales_k.shape[3] != (
            query.shape[1] // batch.group_size
        ):
            raise ValueError("scale dimension mismatch")
        lib = _native.load()
        table = None
        if block_table is not None:
            table = backend._table(block_table, batch.packed_k.shape[0], query.device)
        desc = backend.describe(query, batch, sm_scale, 0 if table is None else table.numel())
        desc.out_query_dtype = int(typed)
        pk, pv = batch.packed_k.contiguous(), batch.packed_v.contiguous()
        sk, sv = batch.scales_k.contiguous(), batch.scales_v.contiguous()
        valid = batch.valid_tokens.contiguous()
        self._need, kern = backend._plan(lib, desc)
        name = _native.KERNEL_NAMES[kern]
        # the library's AUTO demotion for buffers the faster kernels cannot load
        if name == "staged" and not backend._staged_aligned(pk, pv, sk, sv):
            name = "mfma"
        if name == "mfma" and not backend._mfma_aligned(batch.bits, pk, pv, sk, sv):
            name = "general"
        self.kernel = name
        self._backend = backend
        self._keep = (pk, pv, sk, sv, valid, table)
        self._desc = desc
        self._desc_ref = ctypes.byref(desc)
        self._fn = lib.kvssd_hip_fused_decode
        # the same entry point without ctypes' per-argument conversions
        # (~1.5 us a call), when the CPython module built with the library is there
        fast = _native.fused_decode_fast()
        self._fast, self._entry = fast if fast is not None else (None, None)
        self._desc_addr = ctypes.addressof(desc)
        self._ptrs = (_ptr(pk), _ptr(pv), _ptr(sk), _ptr(sv), _ptr(valid), _ptr(table))
        self._device = query.device
        self._index = _index(query.device)
        self._qshape = tuple(query.shape)
        self._qsize = torch.Size(self._qshape)
        self._qdtype = query.dtype
        self._out_shape = (query.shape[0], query.shape[1])
        self._out_dtype = query.dtype if typed else torch.float32
        # per stream: [workspace pointer, workspace bytes, out row pointers,
        # lse row pointers, next row, out rows, lse rows, workspace]
        self._slots: dict[int, list] = {}

    def matches(self, query: torch.Tensor) -> bool:
        """Whether ``query`` has the prepared shape and dtype and sits on the prepared device."""
        return query.dtype is self._qdtype and query.shape == self._qsize and query.get_device() == self._index

    def __call__(self, query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        if not self.matches(query):
            raise ValueError(
                f"query {tuple(query.shape)} {query.dtype} on {query.device} does not match the prepared decode "
                f"({self._qshape} {self._qdtype} on {self._device})"
            )
        return self._call(query)

    def try_call(self, query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor] | None:
        """``self(query)``, or None (nothing launched) when the query does not match."""
        return self._call(query) if self.matches(query) else None

    def _call(self, query: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        q = query if query.is_contiguous() else query.contiguous()
        if _CURRENT_DEVICE() != self._index:
            with torch.cuda.device(self._index):
                return self._launch(q)
        return self._launch(q)

    def _slot(self, handle: int, old: list | None) -> list:
        """A stream's workspace (kept) and a fresh block of output rows."""
        if old is None:
            if len(self._slots) >= self._MAX_STREAMS:
                self._slots.pop(next(iter(self._slots)))
            work = torch.empty((max(self._need, 1),), dtype=torch.uint8, device=self._device)
        else:
            work = old[7]
        outs = torch.empty((self._ROWS, *self._out_shape), dtype=self._out_dtype, device=self._device).unbind(0)
        lses = torch.empty((self._ROWS, self._out_shape[0]), dtype=torch.float32, device=self._device).unbind(0)
        slot = [
            work.data_ptr(), work.numel(), [t.data_ptr() for t in outs], [t.data_ptr() for t in lses], 0, outs, lses,
            work,
        ]
        self._slots[handle] = slot
        return slot

    def _launch(self, q: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        handle = current_stream_handle(self._index)
        slot = self._slots.get(handle)
        if slot is None or slot[4] == self._ROWS:
            slot = self._slot(handle, slot)
        i = slot[4]
        slot[4] = i + 1
        if self._fast is not None:
            rc = self._fast(
                self._entry, self._desc_addr, q.data_ptr(), *self._ptrs, slot[2][i], slot[3][i], slot[0], slot[1], handle
            )
        else:
            rc = self._fn(self._desc_ref, q.data_ptr(), *self._ptrs, slot[2][i], slot[3][i], slot[0], slot[1], handle)
        if rc:
            _native.check(rc, "kvssd_hip_fused_decode")
        self._backend.last_kernel = self.kernel
        return slot[5][i], slot[6][i]
