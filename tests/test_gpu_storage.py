"""The streamed GPU decode over records read from storage: O_DIRECT reads
(page-aligned bounce buffers, then the page-locked staging rows) with the next
chunk's reads in flight while a chunk crosses PCIe, against the oracle; and
record checks deferred to the next decode, so that a loop over layers never
waits for the GPU, still raising decode_record's errors
(src/kvssd/format.py:140-152)."""

from __future__ import annotations

import math
import os
import shutil
import tempfile
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd import KVCacheStore, KVSSDPipeline
from kvssd.format import CacheSpec
from kvssd.selectors import AllBlocks, RecentSinkBlocks
from kvssd.storage.posix import page_aligned_buffer
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
ATOL, RTOL = 2e-3, 1e-2


def supports_o_direct(directory: Path) -> bool:
    probe = directory / ".o_direct_probe"
    try:
        probe.write_bytes(b"\0" * 8192)
        fd = os.open(probe, os.O_RDONLY | os.O_DIRECT)
        try:
            buf = page_aligned_buffer(4096)
            return os.preadv(fd, [memoryview(buf.numpy())], 4096) == 4096
        finally:
            os.close(fd)
    except (OSError, AttributeError):
        return False
    finally:
        probe.unlink(missing_ok=True)


@pytest.fixture
def o_direct_dir(tmp_path: Path):
    # pytest's temporary directory first (tmpfs has no O_DIRECT), then a
    # scratch directory beside the tests
    if supports_o_direct(tmp_path):
        yield tmp_path
        return
    scratch = Path(tempfile.mkdtemp(prefix=".store_", dir=ROOT))
    try:
        if not supports_o_direct(scratch):
            pytest.skip("no O_DIRECT-capable filesystem for the store")
        yield scratch
    finally:
        shutil.rmtree(scratch, ignore_errors=True)


def build(path: Path, storage: str, tokens: int = 2500, bits: int = 4):
    gen = torch.Generator().manual_seed(tokens + 17)
    keys = torch.randn(1, tokens, 8, 128, generator=gen, dtype=torch.float16)
    values = torch.randn(1, tokens, 8, 128, generator=gen, dtype=torch.float16)
    store = KVCacheStore.create(path, keys, values, CacheSpec(1, 8, 128, 128, bits, 32), storage)
    pk, sk, valid = O.quantize_blocks(keys[0].float().numpy(), bits, 32, 128)
    pv, sv, _ = O.quantize_blocks(values[0].float().numpy(), bits, 32, 128)
    return store, (pk, pv, sk, sv, valid)


@pytest.mark.parametrize(("stage_blocks", "io_depth"), [(1, 1), (3, 2), (4, 6)])
def test_streamed_decode_with_o_direct_reads(cuda_device, o_direct_dir: Path, stage_blocks: int, io_depth: int):
    store, (pk, pv, sk, sv, valid) = build(o_direct_dir / "store", "direct")
    assert store.storage_backend.name == "direct"
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(3), dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    with KVSSDPipeline(store, device=cuda_device, io_depth=io_depth, stage_blocks=stage_blocks,
                       attention_backend="hip") as pipe:
        for selector in (AllBlocks(), RecentSinkBlocks(2, 7), RecentSinkBlocks(1, 0)):
            out = pipe.decode(query, 0, selector)
            ids = np.array(selector.select(list(range(20))), np.int32)
            ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, block_table=ids)
            np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    store.close()


def test_deferred_record_checks_raise_at_the_next_decode(cuda_device, tmp_path: Path):
    store, (pk, pv, sk, sv, valid) = build(tmp_path, "buffered", tokens=1024)
    e = store.entry(0, 5)
    with (tmp_path / "blocks.kvssd").open("r+b") as f:
        f.seek(e.offset + 52 + 9000)
        byte = f.read(1)[0]
        f.seek(e.offset + 52 + 9000)
        f.write(bytes([byte ^ 0x40]))
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(4), dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=3, attention_backend="hip",
                       defer_record_checks=True) as pipe:
        pipe.decode(query, 0)  # returns without waiting for the GPU
        with pytest.raises(IOError, match="CRC mismatch for layer=0, block=5"):
            pipe.decode(query, 0, RecentSinkBlocks(1, 2))
        # the check went with the raise; a clean selection decodes correctly
        out = pipe.decode(query, 0, RecentSinkBlocks(2, 2))
        pipe.synchronize()
        ids = np.array(RecentSinkBlocks(2, 2).select(list(range(8))), np.int32)
        ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, block_table=ids)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
        pipe.decode(query, 0, RecentSinkBlocks(0, 3))  # reads block 5 again
        with pytest.raises(IOError, match="block=5"):
            pipe.synchronize()
    store.close()
