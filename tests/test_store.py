"""Store, record format and loader: the reference's tests
(tests/test_store.py:20-59) plus byte equality with the oracle's record."""

from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.format import CacheSpec, decode_record, encode_record
from kvssd.loader import AsyncBlockLoader
from kvssd.quant import dequantize_tensor
from kvssd.store import KVCacheStore
from oracle import oracle as O


def make_store(path: Path, bits: int = 4, storage=None) -> tuple[KVCacheStore, torch.Tensor, torch.Tensor]:
    shape = (2, 19, 2, 32)
    gen = torch.Generator().manual_seed(3)
    keys, values = torch.randn(shape, generator=gen), torch.randn(shape, generator=gen)
    spec = CacheSpec(2, 2, 32, block_tokens=8, bits=bits, group_size=16)
    return KVCacheStore.create(path, keys, values, spec, storage), keys, values


def test_store_round_trip_and_padding(tmp_path: Path) -> None:
    store, keys, _ = make_store(tmp_path)
    block = store.read(1, 2)
    assert block.valid_tokens == 3
    restored = dequantize_tensor(block.key)
    assert torch.mean(torch.abs(restored[:3] - keys[1, 16:])).item() < 0.15
    assert torch.count_nonzero(restored[3:]) == 0
    assert all(entry.offset % 4096 == 0 for entry in store.manifest.entries)


def test_crc_detects_corruption(tmp_path: Path) -> None:
    store, _, _ = make_store(tmp_path)
    entry = store.entry(0, 0)
    data_path = tmp_path / "blocks.kvssd"
    with data_path.open("r+b") as f:
        f.seek(entry.offset + 80)
        old = f.read(1)
        f.seek(entry.offset + 80)
        f.write(bytes([old[0] ^ 0xFF]))
    with pytest.raises(IOError, match="CRC"):
        store.read(0, 0)


def test_async_loader_does_not_alias_recycled_slots(tmp_path: Path) -> None:
    store, _, _ = make_store(tmp_path)
    with AsyncBlockLoader(store, depth=2, pinned=False) as loader:
        blocks = list(loader.iter_blocks(0, [0, 1, 2]))
    snapshots = [x.key.packed.clone() for x in blocks]
    assert [x.block for x in blocks] == [0, 1, 2]
    assert all(torch.equal(x.key.packed, expected) for x, expected in zip(blocks, snapshots))
    direct = [store.read(0, i) for i in range(3)]
    assert all(torch.equal(a.value.packed, b.value.packed) for a, b in zip(blocks, direct))


def test_parallel_reader_closes_its_single_descriptor(tmp_path: Path) -> None:
    store, _, _ = make_store(tmp_path)
    with AsyncBlockLoader(store, depth=3, pinned=False) as loader:
        list(loader.iter_blocks(0, [0, 1, 2]))
    store.close()
    (tmp_path / "blocks.kvssd").unlink()


@pytest.mark.parametrize("bits", [2, 4])
def test_records_match_oracle_bytes_and_reopen(tmp_path: Path, bits: int) -> None:
    store, keys, values = make_store(tmp_path, bits)
    spec = store.spec
    raw = (tmp_path / "blocks.kvssd").read_bytes()
    assert spec.record_bytes == O.record_bytes(2, 32, 8, bits, 16)
    for layer in range(2):
        pk, sk, valid = O.quantize_blocks(keys[layer].numpy(), bits, 16, 8)
        pv, sv, _ = O.quantize_blocks(values[layer].numpy(), bits, 16, 8)
        for b in range(3):
            e = store.entry(layer, b)
            expect = O.encode_record(layer, b, int(valid[b]), bits, 8, 2, 32, 16, sk[b], sv[b], pk[b], pv[b])
            assert raw[e.offset : e.offset + e.length] == expect
    reopened = KVCacheStore.open(tmp_path, "buffered")
    assert reopened.blocks_for_layer(1) == [0, 1, 2]
    assert torch.equal(reopened.read(1, 1).key.packed, store.read(1, 1).key.packed)
    rec, _ = encode_record(store.read(0, 2), spec)
    assert rec == raw[store.entry(0, 2).offset : store.entry(0, 2).offset + spec.record_bytes]


def test_spec_sizes() -> None:
    assert CacheSpec(1, 8, 128, 128, 4, 32).record_bytes == 151552
    assert CacheSpec(1, 8, 128, 128, 2, 32).record_bytes == 86016
    with pytest.raises(ValueError):
        CacheSpec(1, 8, 100, 128, 4, 32).validate()


def test_decode_rejects_layout_mismatch(tmp_path: Path) -> None:
    store, _, _ = make_store(tmp_path)
    e = store.entry(0, 0)
    raw = torch.from_numpy(np.frombuffer((tmp_path / "blocks.kvssd").read_bytes()[e.offset : e.offset + e.length], np.uint8).copy())
    with pytest.raises(ValueError, match="layout"):
        decode_record(raw, CacheSpec(2, 2, 32, block_tokens=8, bits=2, group_size=16))


def test_storage_backends_fail_closed(tmp_path: Path) -> None:
    from kvssd.storage import available_storage_backends, resolve_storage_backend

    make_store(tmp_path)
    names = {s.name: s for s in available_storage_backends(tmp_path / "blocks.kvssd")}
    assert set(names) >= {"gds", "direct", "buffered"} and not names["gds"].available
    with pytest.raises(RuntimeError, match="gds"):
        resolve_storage_backend("gds", tmp_path / "blocks.kvssd")
    with pytest.raises(ValueError, match="unknown storage backend"):
        resolve_storage_backend("nvme-of", tmp_path / "blocks.kvssd")
    assert resolve_storage_backend("buffered", tmp_path / "blocks.kvssd").name == "buffered"


@pytest.mark.parametrize("storage", ["buffered", "direct"])
def test_read_records_copies_raw_bytes_in_order(tmp_path: Path, storage: str) -> None:
    # the record-native read: rows hold the file's record bytes, in the order asked
    store, _, _ = make_store(tmp_path, storage=storage)
    rb = store.spec.record_bytes
    raw = (tmp_path / "blocks.kvssd").read_bytes()
    ids = [2, 0, 1]
    dest = torch.zeros((4, rb), dtype=torch.uint8)
    with AsyncBlockLoader(store, depth=2) as loader:
        loader.read_records(1, ids, dest)
        for row, b in enumerate(ids):
            e = store.entry(1, b)
            assert dest[row].numpy().tobytes() == raw[e.offset : e.offset + e.length]
        assert int(dest[3].count_nonzero()) == 0
        with pytest.raises(ValueError, match="destination"):
            loader.read_records(1, ids, torch.zeros((2, rb), dtype=torch.uint8))
        with pytest.raises(KeyError):
            loader.read_records(1, [7], dest)


def test_host_records_spans_follow_runs() -> None:
    # one H2D span per run of consecutive rows, destination offsets in id order
    from kvssd.staging import HostRecords

    recs = torch.zeros((10, 4096), dtype=torch.uint8)
    host = HostRecords(recs, list(range(100, 110)))
    base = recs.data_ptr()
    spans = host.spans([100, 101, 102, 105, 106, 109, 103], 4096)
    assert spans == [
        (base, 0, 3 * 4096),
        (base + 5 * 4096, 3 * 4096, 2 * 4096),
        (base + 9 * 4096, 5 * 4096, 4096),
        (base + 3 * 4096, 6 * 4096, 4096),
    ]
