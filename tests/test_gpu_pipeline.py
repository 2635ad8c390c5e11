"""GPU pipeline parity (streamed SSD -> pinned staging -> HIP kernels, and
HBM-resident layers) and full-size properties of the 128K-token workload."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd import KVCacheStore, KVSSDPipeline
from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend
from kvssd.format import CacheSpec
from kvssd.selectors import AllBlocks, RecentSinkBlocks
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def build_store(path: Path, tokens: int, bits: int, kvh: int = 8, d: int = 128, bt: int = 128, g: int = 32):
    gen = torch.Generator().manual_seed(tokens + bits)
    keys = torch.randn(1, tokens, kvh, d, generator=gen, dtype=torch.float16)
    values = torch.randn(1, tokens, kvh, d, generator=gen, dtype=torch.float16)
    store = KVCacheStore.create(path, keys, values, CacheSpec(1, kvh, d, bt, bits, g))
    pk, sk, valid = O.quantize_blocks(keys[0].float().numpy(), bits, g, bt)
    pv, sv, _ = O.quantize_blocks(values[0].float().numpy(), bits, g, bt)
    return store, (pk, pv, sk, sv, valid)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("stage_blocks", [1, 3, 8])
def test_streamed_pipeline_matches_oracle(cuda_device, tmp_path: Path, bits: int, stage_blocks: int):
    store, (pk, pv, sk, sv, valid) = build_store(tmp_path, 2500, bits)  # 20 blocks, last one partial
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(1), dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=stage_blocks, attention_backend="hip") as pipe:
        assert pipe.attention_backend.name == "hip"
        for selector in (AllBlocks(), RecentSinkBlocks(1, 4), RecentSinkBlocks(2, 0)):
            out = pipe.decode(query, 0, selector)
            assert out.dtype == torch.float16 and out.device.type == "cuda"
            ids = np.array(selector.select(list(range(20))), np.int32)
            ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, bits, 32, scale, block_table=ids)
            np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def test_resident_pipeline_matches_streamed(cuda_device, tmp_path: Path):
    store, (pk, pv, sk, sv, valid) = build_store(tmp_path, 4096, 4)
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(2), dtype=torch.float16)
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=4, attention_backend="hip") as pipe:
        streamed = pipe.decode(query, 0, RecentSinkBlocks(1, 8))
        pipe.load_resident([0])
        resident = pipe.decode(query, 0, RecentSinkBlocks(1, 8))
        full = pipe.decode(query, 0)
    ids = np.array([0] + list(range(24, 32)), np.int32)
    ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, 1 / math.sqrt(128), block_table=ids)
    np.testing.assert_allclose(resident.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(streamed.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    ref_full, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, 1 / math.sqrt(128))
    np.testing.assert_allclose(full.float().cpu().numpy(), ref_full, atol=ATOL, rtol=RTOL)


class _Ids:
    """A selector returning fixed block ids (any order, repeats allowed)."""

    def __init__(self, ids):
        self.ids = list(ids)

    def select(self, available):
        return list(self.ids)


def test_resident_decode_over_many_selections(cuda_device, tmp_path: Path):
    """More distinct selections than the resident layer keeps device tables for,
    visited twice (tables built, evicted and rebuilt), each against the oracle;
    the whole layer in order takes the no-table form, a permutation of it does not."""
    store, (pk, pv, sk, sv, valid) = build_store(tmp_path, 2500, 4)  # 20 blocks
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(5), dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    q = query.float().numpy()
    selectors = [RecentSinkBlocks(1, r) for r in range(1, 12)] + [AllBlocks(), _Ids(range(19, -1, -1))]
    with KVSSDPipeline(store, device=cuda_device, attention_backend="hip") as pipe:
        pipe.load_resident([0])
        for _ in range(2):
            for sel in selectors:
                out = pipe.decode(query, 0, sel)
                ids = np.array(sel.select(list(range(20))), np.int32)
                ref, _ = O.attention(q, pk, pv, sk, sv, valid, 4, 32, scale, block_table=ids)
                np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
        assert len(pipe._resident[0].tables) <= 8


def test_resident_whole_layer_alternating_queries(cuda_device, tmp_path: Path):
    """Whole-layer decodes of a resident layer re-enter the last call's prepared
    decode only for a query of its shape, dtype and device: queries that change
    dtype, sit on the host, are strided views or have fewer heads each take a
    prepared decode of their own, and every result (kept across later calls)
    matches the oracle in the query's dtype."""
    store, (pk, pv, sk, sv, valid) = build_store(tmp_path, 2500, 4)  # 20 blocks, last one partial
    scale = 1 / math.sqrt(128)
    base = torch.randn(32, 128, generator=torch.Generator().manual_seed(11))
    wide = torch.randn(32, 256, generator=torch.Generator().manual_seed(12))
    queries = [
        base.half().to(cuda_device),
        base.to(cuda_device),
        base.half(),  # host tensor: copied to the device by the pipeline
        base.bfloat16().to(cuda_device),
        wide.half().to(cuda_device)[:, ::2],  # strided view of the same values as below
        wide[:, ::2].contiguous().half().to(cuda_device),
        base[:16].half().to(cuda_device),  # fewer query heads: GQA group of 2
        base.half().to(cuda_device),
    ]
    outs = []
    with KVSSDPipeline(store, device=cuda_device, attention_backend="hip") as pipe:
        pipe.load_resident([0])
        for _ in range(2):
            for q in queries:
                outs.append((q, pipe.decode(q, 0)))
        res = pipe._resident[0]
        assert res.whole is not None and res.whole.matches(queries[-1])
        torch.cuda.synchronize()
    for q, out in outs:
        assert out.dtype == q.dtype and out.device.type == "cuda" and out.shape == q.shape
        ref, _ = O.attention(q.float().cpu().numpy(), pk, pv, sk, sv, valid, 4, 32, scale)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
    # the repeated queries (same values, every call its own output tensor) agree exactly
    n = len(queries)
    for i in range(n):
        assert outs[i][1].data_ptr() != outs[n + i][1].data_ptr()
        assert torch.equal(outs[i][1], outs[n + i][1])
    assert torch.equal(outs[4][1], outs[5][1])


def test_require_cuda_kernel_runs_hip(cuda_device, tmp_path: Path):
    store, _ = build_store(tmp_path, 300, 4)
    with KVSSDPipeline(store, device=cuda_device, require_cuda_kernel=True) as pipe:
        assert pipe.attention_backend.name == "hip"
        out = pipe.decode(torch.randn(32, 128, dtype=torch.float16), 0)
        assert torch.isfinite(out).all()


def synth_packed(tokens: int, bits: int, seed: int, value_scale: float = 1.0, outliers: float = 0.0, qh: int = 32):
    """Quantised synthetic KV [T, 8, 128] in PackedBatch layout (numpy) + fp16 query."""
    gen = torch.Generator().manual_seed(seed)
    k = torch.randn(tokens, 8, 128, generator=gen, dtype=torch.float16)
    v = torch.randn(tokens, 8, 128, generator=gen, dtype=torch.float16)
    q = torch.randn(qh, 128, generator=gen, dtype=torch.float16)
    k, v = (k.float() * value_scale), (v.float() * value_scale)
    if outliers:
        m = torch.rand(k.shape, generator=gen) < outliers
        k[m] *= 8
        v[torch.rand(v.shape, generator=gen) < outliers] *= 8
    pk, sk, valid = O.quantize_blocks(k.half().float().numpy(), bits, 32, 128)
    pv, sv, _ = O.quantize_blocks(v.half().float().numpy(), bits, 32, 128)
    return q, (pk, pv, sk, sv, valid)


@pytest.mark.parametrize(("bits", "value_scale", "outliers"), [(4, 0.5, 0.0), (2, 1.0, 0.05)])
def test_full_size_128k_tokens(cuda_device, bits, value_scale, outliers):
    # the 131072-token INT4 (x0.5 values) and INT2 (5% x8 outliers) workloads:
    # parity with the oracle at full size, plus the size-independent split property
    q, (pk, pv, sk, sv, valid) = synth_packed(131072, bits, 7, value_scale, outliers)
    scale = 1 / math.sqrt(128)
    ref_out, ref_lse = O.attention(q.float().numpy(), pk, pv, sk, sv, valid, bits, 32, scale, threads=16)
    dev = cuda_device
    query = q.to(dev)
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in (pk, pv, sk, sv, valid)), bits, 32)
    for kernel in ["general", "mfma", "staged"]:
        backend = HipAttentionBackend(kernel)
        out, lse = backend.run(query, batch, scale)
        np.testing.assert_allclose(out.cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL)
        # any split of the block range merges back to the one-call result
        a_out, a_lse = backend.run(query, PackedBatch(*(x[:333] for x in (batch.packed_k, batch.packed_v, batch.scales_k, batch.scales_v, batch.valid_tokens)), bits, 32), scale)
        b_out, b_lse = backend.run(query, PackedBatch(*(x[333:] for x in (batch.packed_k, batch.packed_v, batch.scales_k, batch.scales_v, batch.valid_tokens)), bits, 32), scale)
        backend.merge_chunks(a_out, a_lse, b_out, b_lse)
        torch.testing.assert_close(a_out, out, atol=1e-4, rtol=1e-3)
        torch.testing.assert_close(a_lse, lse, atol=1e-4, rtol=1e-4)


def test_sparse_selection_262k_tokens(cuda_device):
    # 262144 tokens, GQA 8, RecentSinkBlocks(1, 32) -> 33 non-contiguous blocks
    q, (pk, pv, sk, sv, valid) = synth_packed(262144, 4, 11, qh=64)
    ids = RecentSinkBlocks(1, 32).select(list(range(2048)))
    assert ids == [0] + list(range(2016, 2048))
    table = np.array(ids, np.int32)
    scale = 1 / math.sqrt(128)
    ref_out, ref_lse = O.attention(q.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, block_table=table)
    dev = cuda_device
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in (pk, pv, sk, sv, valid)), 4, 32)
    for kernel in ["general", "mfma", "staged"]:
        out, lse = HipAttentionBackend(kernel).run(q.to(dev), batch, scale, block_table=ids)
        np.testing.assert_allclose(out.cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("stage_blocks", [2, 5])
def test_host_resident_layer_matches_oracle(cuda_device, tmp_path: Path, stage_blocks: int):
    # raw records kept in page-locked host memory: chunks cross PCIe in runs of
    # consecutive records and are gathered + CRC-checked on the GPU
    store, (pk, pv, sk, sv, valid) = build_store(tmp_path, 2500, 4)
    query = torch.randn(32, 128, generator=torch.Generator().manual_seed(4), dtype=torch.float16)
    scale = 1 / math.sqrt(128)
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=stage_blocks, attention_backend="hip") as pipe:
        pipe.load_host_resident([0])
        for selector in (AllBlocks(), RecentSinkBlocks(3, 6), RecentSinkBlocks(1, 0)):
            out = pipe.decode(query, 0, selector)
            ids = np.array(selector.select(list(range(20))), np.int32)
            ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, block_table=ids)
            np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
        # HBM residency built from the host tier gives the same answer
        pipe.load_resident([0])
        out = pipe.decode(query, 0, RecentSinkBlocks(3, 6))
        ids = np.array(RecentSinkBlocks(3, 6).select(list(range(20))), np.int32)
        ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, block_table=ids)
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)


def corrupt(path: Path, store: KVCacheStore, block: int, at: int, value: bytes) -> None:
    e = store.entry(0, block)
    with (path / "blocks.kvssd").open("r+b") as f:
        f.seek(e.offset + at)
        f.write(value)


def test_streamed_decode_raises_on_corrupt_records(cuda_device, tmp_path: Path):
    # a flipped payload byte raises decode_record's IOError from the GPU CRC
    # check; a bad magic raises its ValueError; unselected blocks are not read
    store, _ = build_store(tmp_path, 1024, 4)  # 8 blocks
    query = torch.randn(32, 128, dtype=torch.float16)
    corrupt(tmp_path, store, 5, 52 + 20000, b"\x5a")
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=3, attention_backend="hip") as pipe:
        with pytest.raises(IOError, match="CRC mismatch for layer=0, block=5"):
            pipe.decode(query, 0)
        assert torch.isfinite(pipe.decode(query, 0, RecentSinkBlocks(2, 1))).all()
        with pytest.raises(IOError, match="block=5"):
            pipe.load_resident([0])
        pipe.load_host_resident([0])
        with pytest.raises(IOError, match="block=5"):
            pipe.decode(query, 0, RecentSinkBlocks(0, 3))
    corrupt(tmp_path, store, 1, 0, b"KVSSD999")
    with KVSSDPipeline(store, device=cuda_device, stage_blocks=4, attention_backend="hip") as pipe:
        with pytest.raises(ValueError, match="invalid KVSSD record header"):
            pipe.decode(query, 0, RecentSinkBlocks(2, 0))


def test_host_staged_1m_tokens(cuda_device):
    # the 1,048,576-token host-staged workload: raw records of the layer in
    # page-locked host memory, streamed in 64-record chunks (one H2D each),
    # gathered, CRC-checked, decoded and merged on the GPU; parity with the
    # oracle over the same records parsed on the host
    from kvssd import records_hip as R
    from kvssd.staging import HostRecords, RecordStager

    spec = CacheSpec(1, 8, 128, 128, 4, 32)
    nb, dev = 8192, cuda_device
    gen = torch.Generator(device=dev).manual_seed(13)
    keys = torch.randn(nb * 128, 8, 128, generator=gen, device=dev, dtype=torch.float16)
    values = torch.randn(nb * 128, 8, 128, generator=gen, device=dev, dtype=torch.float16)
    query = torch.randn(32, 128, generator=gen, device=dev, dtype=torch.float16)
    records, _ = R.encode_records(keys, values, spec, layer=0)
    del keys, values
    pinned = torch.empty(records.shape, dtype=torch.uint8, pin_memory=True)
    pinned.copy_(records)
    del records
    scale = 1 / math.sqrt(128)
    backend = HipAttentionBackend()
    stager = RecordStager(spec, dev, 64, backend, torch.cuda.Stream(dev), torch.cuda.Stream(dev))
    ids = list(range(nb))
    out, lse = stager.run(query, scale, 0, ids, stager.host_fill(HostRecords(pinned, ids)))
    torch.cuda.synchronize()

    raw = pinned.numpy()
    s, pb = 128 * 8 * 4 * 2, 128 * 8 * 64
    base = 52
    sk = np.ascontiguousarray(raw[:, base : base + s]).view(np.float16).reshape(nb, 128, 8, 4)
    sv = np.ascontiguousarray(raw[:, base + s : base + 2 * s]).view(np.float16).reshape(nb, 128, 8, 4)
    pk = np.ascontiguousarray(raw[:, base + 2 * s : base + 2 * s + pb]).reshape(nb, 128, 8, 64)
    pv = np.ascontiguousarray(raw[:, base + 2 * s + pb : base + 2 * s + 2 * pb]).reshape(nb, 128, 8, 64)
    valid = np.full(nb, 128, np.int32)
    ref_out, ref_lse = O.attention(query.float().cpu().numpy(), pk, pv, sk, sv, valid, 4, 32, scale, threads=16)
    np.testing.assert_allclose(out.cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("bits", [2, 4])
def test_store_created_on_gpu_is_byte_identical(cuda_device, tmp_path: Path, bits: int):
    # device keys / values are encoded on the GPU; the data file and the
    # manifest equal those of the CPU quantiser, and the pipeline reads them
    gen = torch.Generator().manual_seed(31 + bits)
    keys = torch.randn(2, 1000, 8, 128, generator=gen, dtype=torch.float16)
    values = torch.randn(2, 1000, 8, 128, generator=gen, dtype=torch.float16)
    spec = CacheSpec(2, 8, 128, 128, bits, 32)
    cpu = KVCacheStore.create(tmp_path / "cpu", keys, values, spec)
    gpu = KVCacheStore.create(tmp_path / "gpu", keys.to(cuda_device), values.to(cuda_device), spec)
    assert (tmp_path / "cpu" / "blocks.kvssd").read_bytes() == (tmp_path / "gpu" / "blocks.kvssd").read_bytes()
    assert cpu.manifest.entries == gpu.manifest.entries
    query = torch.randn(32, 128, generator=gen, dtype=torch.float16)
    with KVSSDPipeline(gpu, device=cuda_device, stage_blocks=3, attention_backend="hip") as pipe:
        out = pipe.decode(query, 1)
    pk, sk, valid = O.quantize_blocks(keys[1].float().numpy(), bits, 32, 128)
    pv, sv, _ = O.quantize_blocks(values[1].float().numpy(), bits, 32, 128)
    ref, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, bits, 32, 1 / math.sqrt(128))
    np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL)
