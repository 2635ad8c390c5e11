"""Attention-backend registry and the PackedBatch contract, on the CPU.

Pins the behaviour of src/kvssd/backends/registry.py:23-68 and
src/kvssd/backends/base.py:29-55 that callers rely on: ``auto`` picks the
portable backend off the GPU, explicit names fail closed with the backend's
reason, unknown names list the choices, instances are probed, and a malformed
batch is rejected with the reference's messages.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.attention import packed_attention
from kvssd.backends import (
    BackendAvailability,
    PackedBatch,
    available_attention_backends,
    register_attention_backend,
    resolve_attention_backend,
)
from kvssd.backends.hip import HipAttentionBackend
from kvssd.backends.reference import ReferenceAttentionBackend
from kvssd.format import CacheSpec
from kvssd.pipeline import KVSSDPipeline
from kvssd.store import KVCacheStore
from oracle import oracle as O


@pytest.mark.parametrize("requested", ["auto", "AUTO ", None])
def test_auto_off_the_gpu_is_the_portable_backend(requested):
    assert resolve_attention_backend(requested, "cpu").name == "reference"


def test_listing_reports_every_builtin_with_a_reason():
    states = {s.name: s for s in available_attention_backends(torch.device("cpu"))}
    assert {"hip", "cuda", "triton", "reference"} <= set(states)
    assert states["reference"].available and not states["reference"].accelerated
    for name in ("hip", "cuda", "triton"):
        assert not states[name].available and states[name].reason
        assert states[name].device_type == "cpu"


@pytest.mark.parametrize(("name", "reason"), [("hip", "ROCm GPU"), ("cuda", "CUDA extension requires"), ("triton", "")])
def test_explicit_names_fail_closed_with_their_reason(name, reason):
    with pytest.raises(RuntimeError, match=f"attention backend '{name}' unavailable: .*{reason}"):
        resolve_attention_backend(name, "cpu")


def test_unknown_name_lists_the_choices():
    with pytest.raises(ValueError) as err:
        resolve_attention_backend("imaginary", "cpu")
    msg = str(err.value)
    assert msg.startswith("unknown attention backend 'imaginary'")
    for name in ("auto", "hip", "cuda", "reference", "triton"):
        assert name in msg


def test_instances_are_probed_not_trusted():
    ref = ReferenceAttentionBackend()
    assert resolve_attention_backend(ref, "cpu") is ref
    with pytest.raises(RuntimeError, match="'hip' unavailable"):
        resolve_attention_backend(HipAttentionBackend(), "cpu")


class _Echo:
    """A third-party backend: always available, returns zeros."""

    name = "echo"

    def probe(self, device):
        return BackendAvailability(self.name, True, False, False, "test backend", torch.device(device).type)

    def run(self, query, batch, sm_scale):
        return torch.zeros(query.shape), torch.zeros(query.shape[0])


def test_registration_by_name():
    for bad in ("", "  ", "auto", "Auto"):
        with pytest.raises(ValueError, match="cannot be 'auto'"):
            register_attention_backend(bad, _Echo)
    register_attention_backend(" Echo-Test ", _Echo)
    assert isinstance(resolve_attention_backend("echo-test", "cpu"), _Echo)
    assert "echo" in {s.name for s in available_attention_backends("cpu")}


def _store(path: Path):
    # 3 kv heads, GQA 2, 6 blocks of 8 tokens, the last one partial
    gen = torch.Generator().manual_seed(2024)
    keys = torch.randn(1, 45, 3, 32, generator=gen)
    values = torch.randn(1, 45, 3, 32, generator=gen)
    spec = CacheSpec(1, 3, 32, block_tokens=8, bits=4, group_size=8)
    return KVCacheStore.create(path, keys, values, spec), keys, values


def test_explicit_and_automatic_portable_backend_agree_with_the_oracle(tmp_path: Path):
    store, keys, values = _store(tmp_path)
    blocks = [store.read(0, b) for b in store.blocks_for_layer(0)]
    query = torch.randn(6, 32, generator=torch.Generator().manual_seed(1))
    named = packed_attention(query, blocks, attention_backend="reference")
    auto = packed_attention(query, blocks)
    assert torch.equal(named, auto)
    pk, sk, valid = O.quantize_blocks(keys[0].numpy(), 4, 8, 8)
    pv, sv, _ = O.quantize_blocks(values[0].numpy(), 4, 8, 8)
    assert valid.tolist() == [8, 8, 8, 8, 8, 5]
    expect, _ = O.attention(query.numpy(), pk, pv, sk, sv, valid, 4, 8, 1 / math.sqrt(32))
    np.testing.assert_allclose(auto.numpy(), expect, atol=2e-5, rtol=2e-5)
    store.close()


def test_pipeline_reports_and_guards_its_backend(tmp_path: Path):
    store, _, _ = _store(tmp_path)
    with KVSSDPipeline(store, device="cpu", attention_backend="reference") as pipe:
        assert pipe.attention_backend.name == "reference"
    with pytest.raises(ValueError, match="conflicts"):
        KVSSDPipeline(store, device="cpu", require_cuda_kernel=True, attention_backend="reference")
    blocks = [store.read(0, 0)]
    with pytest.raises(RuntimeError, match="'hip' unavailable"):
        packed_attention(torch.randn(6, 32), blocks, require_cuda_kernel=True)
    store.close()


def test_packed_batch_validation_messages():
    q = torch.randn(4, 32)
    kp = torch.zeros(2, 8, 2, 16, dtype=torch.uint8)
    ks = torch.zeros(2, 8, 2, 2, dtype=torch.float16)
    valid = torch.tensor([8, 5], dtype=torch.int32)
    PackedBatch(kp, kp, ks, ks, valid, 4, 16).validate(q)
    cases = [
        (PackedBatch(kp, kp, ks, ks, valid, 3, 16), q, "bits must be 2 or 4"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 5), q, "group_size must divide head_dim"),
        (PackedBatch(kp, kp[:1], ks, ks, valid, 4, 16), q, "packed KV must match"),
        (PackedBatch(kp, kp, ks, ks[:1], valid, 4, 16), q, "KV scales must match"),
        (PackedBatch(kp, kp, ks, ks, valid[:1], 4, 16), q, "one count per block"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(3, 32), "divisible by KV heads"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(4, 64), "packed dimension"),
        (PackedBatch(kp, kp, ks, ks, valid, 4, 16), torch.randn(4, 32, 1), r"query must be \[query_heads, head_dim\]"),
    ]
    for batch, query, msg in cases:
        with pytest.raises(ValueError, match=msg):
            batch.validate(query)
