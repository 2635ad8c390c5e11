"""vLLM block codec on the GPU (reference: src/kvssd/integrations/vllm_codec.py:18-102).

The reference compresses a vLLM KV block held in CPU memory into a
``KVVLLM02`` record and decompresses it into a CPU destination.  These are the
same two functions for blocks that live in (or go to) device memory, with the
same record bytes and the same exceptions:

* :func:`encode_vllm_block` -- the block's values (fp16 / bf16 / fp32, any
  shape, taken as one flat vector) are quantised, packed and checksummed on the
  GPU straight into the record; only the compressed record has to cross PCIe
  towards the offload tier;
* :func:`decode_vllm_block` -- the header is parsed and checked on the host
  (truncation, magic / version, dtype code, payload layout, destination size:
  the reference's ValueErrors); the payload (a host record is copied to the
  device first) is CRC-checked and dequantised on the GPU into the
  destination.  A CRC mismatch raises IOError as the reference does; the
  destination then holds the unverified values, where the reference leaves it
  untouched.
"""

from __future__ import annotations

import ctypes
import struct
import zlib
from dataclasses import dataclass

import torch

from . import _native
from .quant import _check

MAGIC = b"KVVLLM02"
HEADER = struct.Struct("<8sBBBBIIQI")
_DTYPE_TO_CODE = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
_CODE_TO_DTYPE = {value: key for key, value in _DTYPE_TO_CODE.items()}
_NATIVE_DTYPE = {torch.float16: _native.DTYPE_F16, torch.bfloat16: _native.DTYPE_BF16, torch.float32: _native.DTYPE_F32}


@dataclass(frozen=True)
class VLLMRecordInfo:
    bits: int
    group_size: int
    dtype: torch.dtype
    elements: int
    payload_bytes: int


def _sizes(elements: int, bits: int, group_size: int) -> tuple[int, int]:
    rec, scratch = ctypes.c_size_t(0), ctypes.c_size_t(0)
    rc = _native.load().kvssd_hip_vllm_sizes(elements, bits, group_size, ctypes.byref(rec), ctypes.byref(scratch))
    _native.check(rc, "kvssd_hip_vllm_sizes")
    return int(rec.value), int(scratch.value)


def _stream() -> int:
    return _native.stream_handle(torch.cuda.current_stream())


def encode_vllm_block(values: torch.Tensor, *, bits: int, group_size: int) -> torch.Tensor:
    """The ``KVVLLM02`` record of a block held on the GPU, as a device uint8
    tensor (byte-identical to encode_vllm_block over the block's memory)."""
    if values.device.type != "cuda":
        raise TypeError("encode_vllm_block expects a device tensor")
    dtype = values.dtype
    if dtype not in _DTYPE_TO_CODE:
        raise KeyError(dtype)  # the reference's _DTYPE_TO_CODE[dtype] lookup
    flat = values.contiguous().view(-1)
    if flat.numel() % group_size:
        raise ValueError(f"vLLM block has {flat.numel()} values, not divisible by group_size={group_size}")
    _check(flat, bits, group_size)
    rec_bytes, scratch_bytes = _sizes(flat.numel(), bits, group_size)
    record = torch.empty(rec_bytes, dtype=torch.uint8, device=flat.device)
    scratch = torch.empty(scratch_bytes, dtype=torch.uint8, device=flat.device)
    crc = torch.empty(1, dtype=torch.int32, device=flat.device)
    rc = _native.load().kvssd_hip_vllm_encode(
        flat.data_ptr(),
        _NATIVE_DTYPE[dtype],
        flat.numel(),
        bits,
        group_size,
        record.data_ptr(),
        crc.data_ptr(),
        scratch.data_ptr(),
        scratch_bytes,
        _stream(),
    )
    _native.check(rc, "kvssd_hip_vllm_encode")
    return record


def decode_vllm_block(raw: torch.Tensor, destination: torch.Tensor) -> VLLMRecordInfo:
    """Decode a record (uint8 tensor on the host or the device) into the device
    tensor ``destination``, whose bytes are taken as the record's dtype."""
    if raw.dtype != torch.uint8 or raw.dim() != 1:
        raise TypeError("raw record must be a 1-D uint8 tensor")
    if destination.device.type != "cuda" or not destination.is_contiguous():
        raise TypeError("destination must be a contiguous device tensor")
    if raw.numel() < HEADER.size:
        raise ValueError("truncated KVSSD vLLM record")
    head = bytes(raw[: HEADER.size].cpu().numpy())
    magic, version, bits, dtype_code, _, group_size, elements, payload_bytes, crc = HEADER.unpack_from(head)
    if magic != MAGIC or version != 1:
        raise ValueError("invalid KVSSD vLLM record header")
    try:
        dtype = _CODE_TO_DTYPE[dtype_code]
    except KeyError as exc:
        raise ValueError(f"unsupported KVSSD vLLM dtype code {dtype_code}") from exc
    payload = raw[HEADER.size : HEADER.size + payload_bytes]
    if payload.numel() != payload_bytes:
        raise ValueError("truncated KVSSD vLLM payload")

    def host_crc_error() -> None:
        # the reference checks the CRC before the layout and the destination:
        # keep that order on the error paths
        if zlib.crc32(bytes(payload.cpu().numpy())) != crc:
            raise IOError("KVSSD vLLM block CRC mismatch")

    scale_count = elements // group_size if group_size else 0
    if group_size == 0 or scale_count * 2 + elements * bits // 8 != payload_bytes:
        host_crc_error()
        raise ValueError("KVSSD vLLM payload layout is inconsistent")
    item = torch.empty((), dtype=dtype).element_size()
    nbytes = destination.numel() * destination.element_size()
    if nbytes % item:
        host_crc_error()
        raise ValueError(f"block byte length {nbytes} is not divisible by {dtype}")
    if nbytes // item != elements:
        host_crc_error()
        raise ValueError(f"destination has {nbytes // item} values, record requires {elements}")
    if elements == 0:
        host_crc_error()
        return VLLMRecordInfo(bits, group_size, dtype, elements, payload_bytes)
    if bits not in (2, 4) or elements % group_size or group_size % (8 // bits):
        host_crc_error()
        raise ValueError("KVSSD vLLM payload layout is inconsistent")
    dev = destination.device
    payload = payload.to(dev, non_blocking=payload.is_pinned()).contiguous()
    _, scratch_bytes = _sizes(elements, bits, group_size)
    scratch = torch.empty(scratch_bytes, dtype=torch.uint8, device=dev)
    status = torch.empty(1, dtype=torch.int32, device=dev)
    rc = _native.load().kvssd_hip_vllm_decode(
        payload.data_ptr(),
        elements,
        bits,
        group_size,
        crc,
        _NATIVE_DTYPE[dtype],
        destination.data_ptr(),
        status.data_ptr(),
        scratch.data_ptr(),
        scratch_bytes,
        _stream(),
    )
    _native.check(rc, "kvssd_hip_vllm_decode")
    if int(status.item()) != 0:
        raise IOError("KVSSD vLLM block CRC mismatch")
    return VLLMRecordInfo(bits, group_size, dtype, elements, payload_bytes)
