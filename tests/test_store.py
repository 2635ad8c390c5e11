"""Store, record format, storage backends and loader on the CPU: padding,
CRC and header checks of decode_record (src/kvssd/format.py:134-177), the
prefetcher's slot reuse and descriptor lifecycle, byte equality with the
oracle's records, and the record-native reads the GPU pipeline uses."""

import os
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


def test_padded_tail_block_decodes_to_zeros(tmp_path: Path) -> None:
    # 19 tokens in blocks of 8: blocks 0, 1 full, block 2 holds 3 tokens and
    # 5 zero rows (src/kvssd/store.py:47-53); every record starts on a 4 KiB
    # boundary; the stored codes are exactly the oracle's
    store, keys, _ = make_store(tmp_path)
    assert [store.read(1, b).valid_tokens for b in range(3)] == [8, 8, 3]
    assert all(e.offset % 4096 == 0 and e.length % 4096 == 0 for e in store.manifest.entries)
    tail = store.read(1, 2)
    back = dequantize_tensor(tail.key)
    assert torch.count_nonzero(back[3:]) == 0
    assert torch.count_nonzero(tail.key.scales[3:]) == 0
    pk, sk, _ = O.quantize_blocks(keys[1].numpy(), 4, 16, 8)
    assert np.array_equal(tail.key.packed.numpy(), pk[2])
    assert np.array_equal(tail.key.scales.numpy().view(np.uint16), sk[2].view(np.uint16))


@pytest.mark.parametrize("at", [52, 53, 52 + 70, 52 + 300, 52 + 639])  # payload: 640 bytes after the header
def test_any_payload_byte_flip_fails_the_crc(tmp_path: Path, at: int) -> None:
    store, _, _ = make_store(tmp_path)
    entry = store.entry(1, 1)
    with (tmp_path / "blocks.kvssd").open("r+b") as f:
        f.seek(entry.offset + at)
        byte = f.read(1)[0]
        f.seek(entry.offset + at)
        f.write(bytes([byte ^ 0x10]))
    with pytest.raises(IOError, match="CRC mismatch for layer=1, block=1"):
        store.read(1, 1)
    store.read(1, 0)  # neighbours are untouched


def test_corrupt_header_is_a_value_error(tmp_path: Path) -> None:
    store, _, _ = make_store(tmp_path)
    with (tmp_path / "blocks.kvssd").open("r+b") as f:
        f.seek(store.entry(0, 2).offset)
        f.write(b"KVSSD002")
    with pytest.raises(ValueError, match="invalid KVSSD record header"):
        store.read(0, 2)


def test_prefetched_blocks_survive_slot_reuse(tmp_path: Path) -> None:
    # one slot, so every block after the first is read into recycled memory;
    # blocks already handed out must keep their own bytes
    store, _, _ = make_store(tmp_path)
    order = [2, 0, 1, 1, 0, 2]
    with AsyncBlockLoader(store, depth=1, pinned=False) as loader:
        held = list(loader.iter_blocks(0, order))
    assert [b.block for b in held] == order
    for b in held:
        fresh = store.read(0, b.block)
        assert b.valid_tokens == fresh.valid_tokens
        for mine, theirs in ((b.key, fresh.key), (b.value, fresh.value)):
            assert torch.equal(mine.packed, theirs.packed) and torch.equal(mine.scales, theirs.scales)


def _open_descriptors() -> int:
    return len(os.listdir("/proc/self/fd"))


@pytest.mark.skipif(not os.path.isdir("/proc/self/fd"), reason="needs /proc/self/fd")
@pytest.mark.parametrize("storage", ["buffered", "direct"])
def test_concurrent_readers_share_one_descriptor(tmp_path: Path, storage: str) -> None:
    before = _open_descriptors()
    store, _, _ = make_store(tmp_path, storage=storage)
    with AsyncBlockLoader(store, depth=4, pinned=False) as loader:
        list(loader.iter_blocks(1, [0, 1, 2, 0, 1, 2]))
        assert _open_descriptors() <= before + 1
    store.close()
    assert _open_descriptors() == before
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
