"""The non-streamed accelerated dispatch on the GPU: ``packed_attention`` over
blocks read from a store (src/kvssd/attention.py:105-134) and the low-level
``fused_attention_tensors`` (src/kvssd/attention.py:71-88), through the hip
backend, against the oracle on the 4,096-token INT4 GQA-4 workload (32
blocks of 128 tokens, 8 kv heads, head_dim 128, groups of 32), with and
without needle tokens (tests/needles.py)."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import needles as N
from kvssd.attention import fused_attention_tensors, packed_attention, stack_blocks
from kvssd.format import CacheSpec
from kvssd.store import KVCacheStore
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)
ATOL, RTOL = 2e-3, 1e-2


def make(path: Path, seed: int, needles: bool):
    q16, k, v = N.half_kv(4096 - 51, seed, 1.0, 0.0, 32)  # last block holds 77 tokens
    if needles:
        kb = np.zeros((32 * 128, 8, 128), np.float32)
        vb = np.zeros_like(kb)
        kb[: len(k)], vb[: len(v)] = k, v
        valid = np.array([128] * 31 + [77], np.int32)
        N.plant(kb.reshape(32, 128, 8, 128), vb.reshape(32, 128, 8, 128), q16.float().numpy(), valid, SCALE,
                np.random.default_rng(seed), amp=32.0)
        k, v = kb[: len(k)], vb[: len(v)]
    keys = torch.from_numpy(k).half()[None]
    values = torch.from_numpy(v).half()[None]
    store = KVCacheStore.create(path, keys, values, CacheSpec(1, 8, 128, 128, 4, 32))
    pk, sk, valid = O.quantize_blocks(keys[0].float().numpy(), 4, 32, 128)
    pv, sv, _ = O.quantize_blocks(values[0].float().numpy(), 4, 32, 128)
    return store, q16, (pk, pv, sk, sv, valid)


@pytest.mark.parametrize("needles", [False, True])
def test_packed_attention_through_hip(cuda_device, tmp_path: Path, needles: bool):
    store, q16, (pk, pv, sk, sv, valid) = make(tmp_path, 404, needles)
    assert valid.tolist()[-1] == 77
    blocks = [store.read(0, b) for b in store.blocks_for_layer(0)]
    query = q16.to(cuda_device)
    ref_out, ref_lse = O.attention(q16.float().numpy(), pk, pv, sk, sv, valid, 4, 32, SCALE)
    for kwargs in ({"attention_backend": "hip"}, {"require_cuda_kernel": True}, {}):
        out = packed_attention(query, blocks, **kwargs)
        assert out.dtype == torch.float16 and out.device == query.device and out.shape == (32, 128)
        # the fp16 cast of the output adds at most 2^-11 relative
        np.testing.assert_allclose(out.float().cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
    # selected blocks in any order: the result depends on the set only
    order = [31, 0, 17, 5]
    out = packed_attention(query, [blocks[i] for i in order], attention_backend="hip")
    ref_sel, _ = O.attention(q16.float().numpy(), pk, pv, sk, sv, valid, 4, 32, SCALE,
                             block_table=np.array(order, np.int32))
    np.testing.assert_allclose(out.float().cpu().numpy(), ref_sel, atol=ATOL, rtol=RTOL)
    if needles:
        out32 = packed_attention(query.float(), blocks, attention_backend="hip")
        N.assert_sensitive_match(out32.cpu().numpy(), ref_lse, ref_out, ref_lse, "packed_attention")
    store.close()


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16, torch.float32])
def test_fused_attention_tensors(cuda_device, tmp_path: Path, qdtype):
    store, q16, (pk, pv, sk, sv, valid) = make(tmp_path, 405, True)
    blocks = [store.read(0, b) for b in store.blocks_for_layer(0)]
    kp, vp, ks, vs, va = stack_blocks(blocks, cuda_device)
    query = q16.to(qdtype).to(cuda_device)
    out, lse = fused_attention_tensors(query, kp, vp, ks, vs, va, 4, 32, SCALE)
    assert out.dtype == torch.float32 and lse.dtype == torch.float32 and lse.shape == (32,)
    q = q16.to(qdtype).float().numpy()
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, SCALE)
    N.assert_sensitive_match(out.cpu().numpy(), lse.cpu().numpy(), ref_out, ref_lse, f"fused {qdtype}")
    # one block fewer must not pass the same check
    c_out, c_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, SCALE, block_table=np.arange(31, dtype=np.int32))
    assert N.differs(out.cpu().numpy(), lse.cpu().numpy(), c_out, c_lse)
    with pytest.raises(ValueError, match="bits must be 2 or 4"):
        fused_attention_tensors(query, kp, vp, ks, vs, va, 3, 32, SCALE)
    store.close()
