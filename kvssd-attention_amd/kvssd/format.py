"""Fixed-size KV block record format, v1.

The on-disk layout is the reference's (src/kvssd/format.py:14-177), byte for
byte, so stores written by either implementation open in the other:

* a 52-byte little-endian header ``<8sIIIIIIIIIII``: magic ``KVSSD001``,
  version 1, layer, block, valid tokens, bits, block_tokens, kv_heads,
  head_dim, group_size, payload length, CRC-32 of the payload;
* the payload ``Ks | Vs | Kc | Vc``: fp16 key scales ``[BT, KVH, G]``, fp16
  value scales, packed key codes ``[BT, KVH, PD]``, packed value codes;
* zero padding to the next 4096-byte boundary;
* ``manifest.json`` carrying the ``CacheSpec`` and one ``BlockEntry`` per record.
"""

from __future__ import annotations

import json
import struct
import zlib
from dataclasses import asdict, dataclass
from pathlib import Path

import torch

from .quant import QuantizedTensor

ALIGNMENT = 4096
MAGIC = b"KVSSD001"
HEADER = struct.Struct("<8sIIIIIIIIIII")


def align_up(value: int, alignment: int = ALIGNMENT) -> int:
    return -(-value // alignment) * alignment


@dataclass(frozen=True)
class CacheSpec:
    layers: int
    kv_heads: int
    head_dim: int
    block_tokens: int = 128
    bits: int = 4
    group_size: int = 32

    def validate(self) -> None:
        if min(self.layers, self.kv_heads, self.head_dim, self.block_tokens) <= 0:
            raise ValueError("all cache dimensions must be positive")
        if self.bits not in (2, 4):
            raise ValueError("bits must be 2 or 4")
        if self.group_size <= 0 or self.head_dim % self.group_size:
            raise ValueError("head_dim must be divisible by group_size")

    @property
    def packed_dim(self) -> int:
        return self.head_dim * self.bits // 8

    @property
    def scale_count(self) -> int:
        return self.block_tokens * self.kv_heads * (self.head_dim // self.group_size)

    @property
    def packed_count(self) -> int:
        return self.block_tokens * self.kv_heads * self.packed_dim

    @property
    def payload_bytes(self) -> int:
        # two fp16 scale arrays plus two packed code arrays
        return 4 * self.scale_count + 2 * self.packed_count

    @property
    def record_bytes(self) -> int:
        return align_up(HEADER.size + self.payload_bytes)


@dataclass(frozen=True)
class BlockEntry:
    layer: int
    block: int
    offset: int
    length: int
    valid_tokens: int
    crc32: int


@dataclass
class Manifest:
    spec: CacheSpec
    entries: list[BlockEntry]
    version: int = 1

    def save(self, path: Path) -> None:
        body = {
            "version": self.version,
            "spec": asdict(self.spec),
            "entries": [asdict(entry) for entry in self.entries],
        }
        Path(path).write_text(json.dumps(body, indent=2) + "\n", encoding="utf-8")

    @classmethod
    def load(cls, path: Path) -> "Manifest":
        body = json.loads(Path(path).read_text(encoding="utf-8"))
        return cls(
            spec=CacheSpec(**body["spec"]),
            entries=[BlockEntry(**entry) for entry in body["entries"]],
            version=body["version"],
        )


@dataclass(frozen=True)
class PackedKVBlock:
    layer: int
    block: int
    valid_tokens: int
    key: QuantizedTensor
    value: QuantizedTensor


def _as_bytes(t: torch.Tensor) -> bytes:
    t = t.detach().cpu().contiguous()
    if t.dtype != torch.uint8:
        t = t.view(torch.uint8)
    return t.numpy().tobytes()


def encode_record(block: PackedKVBlock, spec: CacheSpec) -> tuple[bytes, int]:
    """Serialise one padded block; returns (record bytes, payload CRC-32)."""
    expected = (spec.block_tokens, spec.kv_heads, spec.head_dim)
    if block.key.original_shape != expected or block.value.original_shape != expected:
        raise ValueError(f"padded KV block must have shape {expected}")
    payload = b"".join(
        (
            _as_bytes(block.key.scales),
            _as_bytes(block.value.scales),
            _as_bytes(block.key.packed),
            _as_bytes(block.value.packed),
        )
    )
    crc = zlib.crc32(payload)
    header = HEADER.pack(
        MAGIC,
        1,
        block.layer,
        block.block,
        block.valid_tokens,
        spec.bits,
        spec.block_tokens,
        spec.kv_heads,
        spec.head_dim,
        spec.group_size,
        len(payload),
        crc,
    )
    body = header + payload
    return body + bytes(spec.record_bytes - len(body)), crc


def payload_views(raw: torch.Tensor, spec: CacheSpec) -> tuple[torch.Tensor, ...]:
    """Views (ks, vs, kp, vp) into a raw record buffer, shaped like PackedBatch rows."""
    scale_shape = (spec.block_tokens, spec.kv_heads, spec.head_dim // spec.group_size)
    packed_shape = (spec.block_tokens, spec.kv_heads, spec.packed_dim)
    s_bytes = 2 * spec.scale_count
    p_bytes = spec.packed_count
    base = HEADER.size
    ks = raw[base : base + s_bytes].view(torch.float16).reshape(scale_shape)
    vs = raw[base + s_bytes : base + 2 * s_bytes].view(torch.float16).reshape(scale_shape)
    kp = raw[base + 2 * s_bytes : base + 2 * s_bytes + p_bytes].reshape(packed_shape)
    vp = raw[base + 2 * s_bytes + p_bytes : base + 2 * s_bytes + 2 * p_bytes].reshape(packed_shape)
    return ks, vs, kp, vp


def decode_record(raw: torch.Tensor, spec: CacheSpec, verify_crc: bool = True) -> PackedKVBlock:
    """Parse a record held in a contiguous CPU uint8 tensor (views, no copies)."""
    if raw.dtype != torch.uint8 or raw.device.type != "cpu" or not raw.is_contiguous():
        raise TypeError("raw record must be a contiguous CPU uint8 tensor")
    mem = memoryview(raw.numpy())
    magic, version, layer, block, valid, bits, bt, heads, dim, group, payload_len, crc = HEADER.unpack(
        bytes(mem[: HEADER.size])
    )
    if magic != MAGIC or version != 1:
        raise ValueError("invalid KVSSD record header")
    layout = (spec.bits, spec.block_tokens, spec.kv_heads, spec.head_dim, spec.group_size)
    if (bits, bt, heads, dim, group) != layout:
        raise ValueError("record layout does not match manifest")
    if verify_crc and zlib.crc32(mem[HEADER.size : HEADER.size + payload_len]) != crc:
        raise IOError(f"CRC mismatch for layer={layer}, block={block}")
    ks, vs, kp, vp = payload_views(raw, spec)
    shape = (spec.block_tokens, spec.kv_heads, spec.head_dim)
    return PackedKVBlock(
        layer=layer,
        block=block,
        valid_tokens=valid,
        key=QuantizedTensor(kp, ks, shape, spec.bits, spec.group_size),
        value=QuantizedTensor(vp, vs, shape, spec.bits, spec.group_size),
    )
