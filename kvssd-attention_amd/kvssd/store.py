"""Append-only fixed-record KV cache store (reference: src/kvssd/store.py:12-113).

``create`` quantises each layer's padded ``[T, KVH, D]`` tensor in one call and
slices it into records.  Groups run along the last dimension only, so this is
byte-identical to the reference's per-block quantisation (store.py:46-60) while
avoiding one small quantiser call per block.  Keys and values that live on a
GPU are quantised, packed and checksummed there (``records_hip.encode_records``,
one launch pair per layer, byte-identical records); only the finished records
cross PCIe.
"""

from __future__ import annotations

from pathlib import Path

import torch

from .format import BlockEntry, CacheSpec, Manifest, PackedKVBlock, decode_record, encode_record
from .quant import QuantizedTensor, quantize_tensor
from .storage import StorageBackend, resolve_storage_backend

DATA_FILE = "blocks.kvssd"
MANIFEST_FILE = "manifest.json"


class KVCacheStore:
    """Append-only fixed-record KV cache store designed for large sequential SSD reads."""

    def __init__(
        self,
        root: str | Path,
        manifest: Manifest,
        storage_backend: str | StorageBackend | None = None,
    ):
        self.root = Path(root)
        self.manifest = manifest
        self.spec = manifest.spec
        self._entries = {(e.layer, e.block): e for e in manifest.entries}
        by_layer: dict[int, list[int]] = {}
        for e in manifest.entries:
            by_layer.setdefault(e.layer, []).append(e.block)
        self._layer_blocks = {layer: sorted(ids) for layer, ids in by_layer.items()}
        self.storage_backend = resolve_storage_backend(storage_backend, self.root / DATA_FILE)

    @classmethod
    def create(
        cls,
        root: str | Path,
        keys: torch.Tensor,
        values: torch.Tensor,
        spec: CacheSpec,
        storage_backend: str | StorageBackend | None = None,
    ) -> "KVCacheStore":
        """Create a store from [layers, tokens, kv_heads, head_dim] tensors."""
        spec.validate()
        if keys.shape != values.shape or keys.ndim != 4:
            raise ValueError("keys and values must share [layers,tokens,kv_heads,head_dim]")
        if keys.shape[0] != spec.layers or tuple(keys.shape[2:]) != (spec.kv_heads, spec.head_dim):
            raise ValueError("input tensors do not match CacheSpec")
        root = Path(root)
        root.mkdir(parents=True, exist_ok=True)
        tokens = keys.shape[1]
        bt = spec.block_tokens
        n_blocks = -(-tokens // bt)
        block_shape = (bt, spec.kv_heads, spec.head_dim)
        entries: list[BlockEntry] = []
        if keys.device.type == "cuda" or values.device.type == "cuda":
            return cls._create_on_gpu(root, keys, values, spec, storage_backend)
        with (root / DATA_FILE).open("wb") as out:
            for layer in range(spec.layers):
                padded = []
                for src in (keys, values):
                    buf = torch.zeros((n_blocks * bt, spec.kv_heads, spec.head_dim), dtype=src.dtype)
                    buf[:tokens].copy_(src[layer].cpu())
                    padded.append(quantize_tensor(buf, spec.bits, spec.group_size))
                kq, vq = padded
                kp = kq.packed.reshape(n_blocks, bt, spec.kv_heads, spec.packed_dim)
                vp = vq.packed.reshape(n_blocks, bt, spec.kv_heads, spec.packed_dim)
                groups = spec.head_dim // spec.group_size
                ks = kq.scales.reshape(n_blocks, bt, spec.kv_heads, groups)
                vs = vq.scales.reshape(n_blocks, bt, spec.kv_heads, groups)
                for block_id in range(n_blocks):
                    valid = min(bt, tokens - block_id * bt)
                    block = PackedKVBlock(
                        layer,
                        block_id,
                        valid,
                        QuantizedTensor(kp[block_id], ks[block_id], block_shape, spec.bits, spec.group_size),
                        QuantizedTensor(vp[block_id], vs[block_id], block_shape, spec.bits, spec.group_size),
                    )
                    record, crc = encode_record(block, spec)
                    offset = out.tell()
                    out.write(record)
                    entries.append(BlockEntry(layer, block_id, offset, len(record), valid, crc))
        manifest = Manifest(spec=spec, entries=entries)
        manifest.save(root / MANIFEST_FILE)
        return cls(root, manifest, storage_backend)

    @classmethod
    def _create_on_gpu(
        cls,
        root: Path,
        keys: torch.Tensor,
        values: torch.Tensor,
        spec: CacheSpec,
        storage_backend: str | StorageBackend | None,
    ) -> "KVCacheStore":
        from .records_hip import encode_records

        device = keys.device if keys.device.type == "cuda" else values.device
        keys, values = keys.to(device), values.to(device)
        tokens = keys.shape[1]
        rb = spec.record_bytes
        entries: list[BlockEntry] = []
        with (root / DATA_FILE).open("wb") as out:
            for layer in range(spec.layers):
                records, crcs = encode_records(keys[layer], values[layer], spec, layer)
                host = records.cpu()
                crc_list = crcs.cpu().tolist()
                for block_id in range(host.shape[0]):
                    offset = out.tell()
                    out.write(memoryview(host[block_id].numpy()))
                    valid = min(spec.block_tokens, tokens - block_id * spec.block_tokens)
                    entries.append(BlockEntry(layer, block_id, offset, rb, valid, int(crc_list[block_id])))
        manifest = Manifest(spec=spec, entries=entries)
        manifest.save(root / MANIFEST_FILE)
        return cls(root, manifest, storage_backend)

    @classmethod
    def open(cls, root: str | Path, storage_backend: str | StorageBackend | None = None) -> "KVCacheStore":
        root = Path(root)
        manifest = Manifest.load(root / MANIFEST_FILE)
        manifest.spec.validate()
        return cls(root, manifest, storage_backend)

    def entry(self, layer: int, block: int) -> BlockEntry:
        try:
            return self._entries[(layer, block)]
        except KeyError as exc:
            raise KeyError(f"no KV block layer={layer}, block={block}") from exc

    def blocks_for_layer(self, layer: int) -> list[int]:
        return list(self._layer_blocks.get(layer, []))

    def read_into(self, entry: BlockEntry, destination: torch.Tensor) -> None:
        self.storage_backend.read_into(entry, destination)

    def read(self, layer: int, block: int, verify_crc: bool = True) -> PackedKVBlock:
        entry = self.entry(layer, block)
        raw = self.storage_backend.allocate_buffer(entry.length)
        self.read_into(entry, raw)
        if raw.device.type != "cpu":
            raw = raw.cpu()
        return decode_record(raw, self.spec, verify_crc)

    def close(self) -> None:
        self.storage_backend.close()

    def __enter__(self) -> "KVCacheStore":
        return self

    def __exit__(self, *_: object) -> None:
        self.close()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
