"""GPU record codec: the v1 block record (format.py) and the quantiser on HBM.

* :func:`gather_records` -- a span of raw records already in device memory
  becomes the ``PackedBatch`` arrays, with decode_record's header, layout and
  payload CRC-32 checks done on the GPU (reference: src/kvssd/format.py:134-177,
  the loader's payload clones src/kvssd/loader.py:73-91 and the pipeline's
  per-array stacking src/kvssd/pipeline.py:98-108);
* :func:`quantize` -- bit-exact twin of ``quantize_tensor``
  (src/kvssd/quant.py:49-65) for device tensors;
* :func:`encode_records` -- whole records of one layer, quantised and
  checksummed on the GPU (KVCacheStore.create's block loop,
  src/kvssd/store.py:46-63, with encode_record, src/kvssd/format.py:104-131).

Every call is asynchronous on the current stream, as the rest of the library.
"""

from __future__ import annotations

import ctypes

import torch

from . import _native
from .format import CacheSpec
from .quant import QuantizedTensor, _check

_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2, torch.float64: 3}
# status codes of kvssd_hip_gather_records
OK, BAD_HEADER, BAD_LAYOUT, BAD_CRC = 0, 1, 2, 3


def _layout(spec: CacheSpec) -> _native.RecordLayout:
    return _native.RecordLayout(spec.bits, spec.block_tokens, spec.kv_heads, spec.head_dim, spec.group_size)


def _stream() -> int:
    return _native.stream_handle(torch.cuda.current_stream())


def record_bytes(spec: CacheSpec) -> int:
    """``CacheSpec.record_bytes`` as the library computes it."""
    out = ctypes.c_size_t(0)
    _native.check(_native.load().kvssd_hip_record_bytes(ctypes.byref(_layout(spec)), ctypes.byref(out)), "record_bytes")
    return int(out.value)


def _check_out(out: tuple[torch.Tensor, ...], spec: CacheSpec, count: int, dev: torch.device) -> None:
    groups = spec.head_dim // spec.group_size
    pshape = (count, spec.block_tokens, spec.kv_heads, spec.packed_dim)
    sshape = (count, spec.block_tokens, spec.kv_heads, groups)
    want = [
        (pshape, torch.uint8),
        (pshape, torch.uint8),
        (sshape, torch.float16),
        (sshape, torch.float16),
        ((count,), torch.int32),
        ((count,), torch.int32),
    ]
    if len(out) != len(want):
        raise ValueError("out must hold (packed_k, packed_v, scales_k, scales_v, valid, status)")
    for t, (shape, dtype) in zip(out, want):
        if tuple(t.shape) != shape or t.dtype != dtype or t.device != dev or not t.is_contiguous():
            raise ValueError(f"gather output must be a contiguous {dtype} tensor of shape {shape} on {dev}")


def gather_records(
    raw: torch.Tensor,
    spec: CacheSpec,
    count: int,
    stride: int | None = None,
    verify_crc: bool = True,
    out: tuple[torch.Tensor, ...] | None = None,
) -> tuple[torch.Tensor, ...]:
    """(packed_k, packed_v, scales_k, scales_v, valid, status) of ``count``
    records held back to back (``stride`` bytes apart, default
    ``record_bytes``) in the device uint8 tensor ``raw``.  ``status`` holds
    per record OK, BAD_HEADER, BAD_LAYOUT or BAD_CRC; see :func:`raise_for_status`.
    ``out`` supplies the six output tensors (else they are allocated)."""
    stride = spec.record_bytes if stride is None else stride
    if raw.dtype != torch.uint8 or raw.device.type != "cuda" or not raw.is_contiguous():
        raise TypeError("raw records must be a contiguous uint8 device tensor")
    if raw.numel() < count * stride:
        raise ValueError("raw buffer holds fewer than count records")
    dev = raw.device
    if out is not None:
        _check_out(out, spec, count, dev)
        pk, pv, sk, sv, valid, status = out
    else:
        bt, kvh = spec.block_tokens, spec.kv_heads
        pk = torch.empty((count, bt, kvh, spec.packed_dim), dtype=torch.uint8, device=dev)
        pv = torch.empty_like(pk)
        sk = torch.empty((count, bt, kvh, spec.head_dim // spec.group_size), dtype=torch.float16, device=dev)
        sv = torch.empty_like(sk)
        valid = torch.empty(count, dtype=torch.int32, device=dev)
        status = torch.empty(count, dtype=torch.int32, device=dev)
    rc = _native.load().kvssd_hip_gather_records(
        ctypes.byref(_layout(spec)),
        raw.data_ptr(),
        stride,
        count,
        1 if verify_crc else 0,
        pk.data_ptr(),
        pv.data_ptr(),
        sk.data_ptr(),
        sv.data_ptr(),
        valid.data_ptr(),
        status.data_ptr(),
        _stream(),
    )
    _native.check(rc, "kvssd_hip_gather_records")
    return pk, pv, sk, sv, valid, status


def raise_for_status(status: torch.Tensor, layer: int, blocks: list[int]) -> None:
    """Raise decode_record's exception for the first bad record
    (src/kvssd/format.py:140-152): ValueError for a bad header or layout,
    IOError for a CRC mismatch.  Synchronises with ``status``."""
    host = status.cpu().tolist()
    for code, block in zip(host, blocks):
        if code == BAD_HEADER:
            raise ValueError("invalid KVSSD record header")
        if code == BAD_LAYOUT:
            raise ValueError("record layout does not match manifest")
        if code == BAD_CRC:
            raise IOError(f"CRC mismatch for layer={layer}, block={block}")


def quantize(x: torch.Tensor, bits: int, group_size: int = 32) -> QuantizedTensor:
    """``quantize_tensor`` on the GPU, bit-identical (packed codes and fp16 scales)."""
    _check(x, bits, group_size)
    if x.device.type != "cuda":
        raise TypeError("quantize expects a device tensor")
    if x.dtype not in _DTYPES:
        raise TypeError("quantization input must be floating point")
    x = x.contiguous()
    shape = tuple(x.shape)
    d = shape[-1]
    rows = x.numel() // d
    packed = torch.empty((*shape[:-1], d * bits // 8), dtype=torch.uint8, device=x.device)
    scales = torch.empty((*shape[:-1], d // group_size), dtype=torch.float16, device=x.device)
    rc = _native.load().kvssd_hip_quantize(
        x.data_ptr(), _DTYPES[x.dtype], rows, d, bits, group_size, packed.data_ptr(), scales.data_ptr(), _stream()
    )
    _native.check(rc, "kvssd_hip_quantize")
    return QuantizedTensor(packed, scales, shape, bits, group_size)


def encode_records(
    keys: torch.Tensor, values: torch.Tensor, spec: CacheSpec, layer: int, first_block: int = 0
) -> tuple[torch.Tensor, torch.Tensor]:
    """Records of one layer from device keys / values [tokens, KVH, D]: a uint8
    tensor [n, record_bytes] (n = ceil(tokens / block_tokens), the last block
    zero-padded) and the payload CRC-32 of each record (int64 [n])."""
    if keys.shape != values.shape or keys.ndim != 3 or tuple(keys.shape[1:]) != (spec.kv_heads, spec.head_dim):
        raise ValueError("keys and values must be [tokens, kv_heads, head_dim] matching the CacheSpec")
    if keys.dtype != values.dtype or keys.dtype not in _DTYPES:
        raise TypeError("quantization input must be floating point")
    if keys.device.type != "cuda" or values.device != keys.device:
        raise TypeError("encode_records expects device tensors on one device")
    keys, values = keys.contiguous(), values.contiguous()
    tokens = keys.shape[0]
    n = -(-tokens // spec.block_tokens)
    rb = spec.record_bytes
    records = torch.empty((n, rb), dtype=torch.uint8, device=keys.device)
    crcs = torch.empty(n, dtype=torch.int32, device=keys.device)
    rc = _native.load().kvssd_hip_encode_records(
        ctypes.byref(_layout(spec)),
        _DTYPES[keys.dtype],
        keys.data_ptr(),
        values.data_ptr(),
        tokens,
        layer,
        first_block,
        records.data_ptr(),
        crcs.data_ptr(),
        _stream(),
    )
    _native.check(rc, "kvssd_hip_encode_records")
    return records, crcs.to(torch.int64) & 0xFFFFFFFF
