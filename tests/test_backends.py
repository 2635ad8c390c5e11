"""Backend registry and contract: the reference's tests (tests/test_backends.py:25-58)
plus the hip backend's fail-closed behaviour without a GPU."""

from pathlib import Path

import pytest
import torch

from kvssd.attention import packed_attention
from kvssd.backends import PackedBatch, available_attention_backends, resolve_attention_backend
from kvssd.format import CacheSpec
from kvssd.pipeline import KVSSDPipeline
from kvssd.store import KVCacheStore


def make_blocks(path: Path):
    gen = torch.Generator().manual_seed(29)
    shape = (1, 11, 2, 32)
    store = KVCacheStore.create(
        path,
        torch.randn(shape, generator=gen),
        torch.randn(shape, generator=gen),
        CacheSpec(1, 2, 32, block_tokens=8, bits=4, group_size=16),
    )
    return store, [store.read(0, block) for block in store.blocks_for_layer(0)]


def test_cpu_auto_resolves_to_reference() -> None:
    backend = resolve_attention_backend("auto", "cpu")
    assert backend.name == "reference"
    availability = available_attention_backends("cpu")
    assert {item.name for item in availability} >= {"cuda", "reference", "hip"}
    assert next(item for item in availability if item.name == "reference").available


def test_explicit_cuda_fails_closed_without_extension() -> None:
    if torch.cuda.is_available():
        pytest.skip("CPU-only failure contract")
    with pytest.raises(RuntimeError, match="CUDA extension requires"):
        resolve_attention_backend("cuda", "cpu")


def test_explicit_hip_fails_closed_on_cpu() -> None:
    with pytest.raises(RuntimeError, match="attention backend 'hip' unavailable"):
        resolve_attention_backend("hip", "cpu")
    with pytest.raises(RuntimeError, match="unavailable"):
        resolve_attention_backend("triton", "cpu")


def test_explicit_reference_matches_legacy_reference(tmp_path: Path) -> None:
    store, blocks = make_blocks(tmp_path)
    query = torch.randn(4, 32, generator=torch.Generator().manual_seed(31))
    explicit = packed_attention(query, blocks, attention_backend="reference")
    automatic = packed_attention(query, blocks)
    torch.testing.assert_close(explicit, automatic)
    store.close()


def test_pipeline_exposes_selected_backend(tmp_path: Path) -> None:
    store, _ = make_blocks(tmp_path)
    with KVSSDPipeline(store, device="cpu", attention_backend="reference") as pipeline:
        assert pipeline.attention_backend.name == "reference"
    store.close()


def test_require_cuda_kernel_is_the_native_kernel(tmp_path: Path) -> None:
    store, blocks = make_blocks(tmp_path)
    with pytest.raises(ValueError, match="conflicts"):
        KVSSDPipeline(store, device="cpu", require_cuda_kernel=True, attention_backend="reference")
    with pytest.raises(RuntimeError, match="'hip' unavailable"):
        packed_attention(torch.randn(4, 32), blocks, require_cuda_kernel=True)
    store.close()


def test_unknown_backend_reports_choices() -> None:
    with pytest.raises(ValueError, match="unknown attention backend"):
        resolve_attention_backend("imaginary", "cpu")


def test_packed_batch_validation_messages() -> None:
    q = torch.randn(4, 32)
    kp = torch.zeros(2, 8, 2, 16, dtype=torch.uint8)
    ks = torch.zeros(2, 8, 2, 2, dtype=torch.float16)
    valid = torch.tensor([8, 5], dtype=torch.int32)
    PackedBatch(kp, kp, ks, ks, valid, 4, 16).validate(q)
    cases = [
        (PackedBatch(kp, kp, ks, ks, valid, 3, 16), q, "bits"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 5), q, "group_size"),
        (PackedBatch(kp, kp[:1], ks, ks, valid, 4, 16), q, "packed KV"),
        (PackedBatch(kp, kp, ks, ks[:1], valid, 4, 16), q, "scales"),
        (PackedBatch(kp, kp, ks, ks, valid[:1], 4, 16), q, "valid_tokens"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(3, 32), "divisible"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(4, 64), "packed dimension"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(4, 32, 1), "query"),
    ]
    for batch, query, msg in cases:
        with pytest.raises(ValueError, match=msg):
            batch.validate(query)
