"""Attention orchestration on the CPU: the dense reference path, packed
attention through the portable backend, block stacking and the exact chunk
merge, each against the oracle or a float64 computation written out here."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.attention import (
    merge_attention_chunks,
    packed_attention,
    packed_attention_reference,
    reference_attention,
    stack_blocks,
)
from kvssd.backends import PackedBatch
from kvssd.backends.reference import ReferenceAttentionBackend
from kvssd.format import CacheSpec, PackedKVBlock
from kvssd.quant import quantize_tensor
from kvssd.store import KVCacheStore
from oracle import oracle as O


def dense_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """Decode attention written as loops over query heads, in float64."""
    qh = q.shape[0]
    gq = qh // k.shape[1]
    out = np.zeros(q.shape)
    for h in range(qh):
        s = k[:, h // gq].astype(np.float64) @ q[h].astype(np.float64) * scale
        w = np.exp(s - s.max())
        out[h] = w @ v[:, h // gq].astype(np.float64) / w.sum()
    return out


@pytest.mark.parametrize(("qh", "kvh", "t"), [(1, 1, 1), (4, 2, 17), (6, 3, 40), (8, 1, 5)])
def test_reference_attention_against_float64_loops(qh, kvh, t):
    gen = torch.Generator().manual_seed(qh * 100 + t)
    q = torch.randn(qh, 16, generator=gen, dtype=torch.float64)
    k = torch.randn(t, kvh, 16, generator=gen)
    v = torch.randn(t, kvh, 16, generator=gen)
    got = reference_attention(q, k, v, sm_scale=0.3)
    assert got.dtype == torch.float64
    np.testing.assert_allclose(got.numpy(), dense_f64(q.numpy(), k.numpy(), v.numpy(), 0.3), rtol=1e-5, atol=1e-6)
    default = reference_attention(q.half(), k, v)  # 1/sqrt(D), cast to the query dtype
    assert default.dtype == torch.float16
    np.testing.assert_allclose(default.float().numpy(), dense_f64(q.half().numpy(), k.numpy(), v.numpy(), 0.25),
                               rtol=2e-3, atol=2e-3)


def test_reference_attention_shape_errors():
    with pytest.raises(ValueError, match="divisible"):
        reference_attention(torch.randn(3, 8), torch.randn(4, 2, 8), torch.randn(4, 2, 8))
    with pytest.raises(ValueError, match="head_dim mismatch"):
        reference_attention(torch.randn(4, 8), torch.randn(4, 2, 16), torch.randn(4, 2, 16))
    with pytest.raises(ValueError, match=r"expected query \[QH,D\]"):
        reference_attention(torch.randn(4, 8), torch.randn(4, 2, 8), torch.randn(5, 2, 8))


def _blocks(tmp_path: Path, bits: int):
    gen = torch.Generator().manual_seed(50 + bits)
    keys = torch.randn(1, 29, 2, 64, generator=gen)
    values = torch.randn(1, 29, 2, 64, generator=gen)
    store = KVCacheStore.create(tmp_path, keys, values, CacheSpec(1, 2, 64, block_tokens=8, bits=bits, group_size=16))
    return store, [store.read(0, b) for b in store.blocks_for_layer(0)], keys[0], values[0]


@pytest.mark.parametrize("bits", [2, 4])
def test_packed_attention_matches_the_oracle(tmp_path: Path, bits: int):
    store, blocks, keys, values = _blocks(tmp_path, bits)
    query = torch.randn(4, 64, generator=torch.Generator().manual_seed(9))
    got = packed_attention(query, blocks)
    assert got.dtype == query.dtype and got.shape == (4, 64)
    pk, sk, valid = O.quantize_blocks(keys.numpy(), bits, 16, 8)
    pv, sv, _ = O.quantize_blocks(values.numpy(), bits, 16, 8)
    assert valid.tolist() == [8, 8, 8, 5]
    expect, _ = O.attention(query.numpy(), pk, pv, sk, sv, valid, bits, 16, 1 / 8)
    np.testing.assert_allclose(got.numpy(), expect, atol=2e-5, rtol=2e-5)
    # the dequantise-then-attend helper gives the same result
    torch.testing.assert_close(packed_attention_reference(query, blocks), got, atol=1e-6, rtol=1e-6)
    with pytest.raises(ValueError, match="at least one block"):
        packed_attention(query, [])
    store.close()


def test_stack_blocks_keeps_block_order_and_counts(tmp_path: Path):
    store, blocks, _, _ = _blocks(tmp_path, 4)
    order = [blocks[3], blocks[0], blocks[2]]
    kp, vp, ks, vs, valid = stack_blocks(order, torch.device("cpu"))
    assert kp.shape == (3, 8, 2, 32) and ks.shape == (3, 8, 2, 4) and ks.dtype == torch.float16
    assert valid.dtype == torch.int32 and valid.tolist() == [5, 8, 8]
    for i, b in enumerate(order):
        assert torch.equal(kp[i], b.key.packed) and torch.equal(vp[i], b.value.packed)
        assert torch.equal(ks[i], b.key.scales) and torch.equal(vs[i], b.value.scales)
    with pytest.raises(ValueError, match="at least one block"):
        stack_blocks([], torch.device("cpu"))
    store.close()


def _block(tokens: int, bits: int, valid: int, seed: int) -> PackedKVBlock:
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(tokens, 2, 32, generator=g, dtype=torch.float16)
    v = torch.randn(tokens, 2, 32, generator=g, dtype=torch.float16)
    return PackedKVBlock(0, seed, valid, quantize_tensor(k, bits, 8), quantize_tensor(v, bits, 8))


def test_stack_blocks_rejects_blocks_unlike_the_first():
    # the reference's torch.stack raises on a shape mismatch; a broadcastable
    # block (1 token against 8) must not be replicated into the batch
    with pytest.raises(RuntimeError, match="equal size"):
        stack_blocks([_block(8, 4, 8, 1), _block(1, 4, 1, 2)], torch.device("cpu"))
    with pytest.raises(RuntimeError, match="equal size"):
        stack_blocks([_block(8, 4, 8, 1), _block(8, 2, 8, 2)], torch.device("cpu"))


def test_packed_attention_reference_over_unlike_blocks():
    # blocks of different lengths and bit widths: each is dequantised on its
    # own and its valid rows concatenated (src/kvssd/attention.py:34-47);
    # checked against float64 attention over the oracle's dequantisation
    blocks = [_block(8, 4, 6, 1), _block(16, 2, 16, 2), _block(4, 4, 3, 3)]
    q = torch.randn(4, 32, generator=torch.Generator().manual_seed(9), dtype=torch.float16)
    out = packed_attention_reference(q, blocks, 0.2)
    ks, vs = [], []
    for b in blocks:
        for t, dst in ((b.key, ks), (b.value, vs)):
            codes = O.unpack_np(t.packed.numpy(), t.bits, t.original_shape[-1])
            deq = O.dequantize_np(codes, t.scales.numpy(), t.bits, t.group_size)
            dst.append(deq.reshape(t.original_shape)[: b.valid_tokens].astype(np.float64))
    k, v = np.concatenate(ks), np.concatenate(vs)
    qf = q.double().numpy()
    want = np.zeros((4, 32))
    for h in range(4):
        s = 0.2 * (k[:, h // 2] @ qf[h])
        p = np.exp(s - s.max())
        want[h] = (p / p.sum()) @ v[:, h // 2]
    assert out.dtype == torch.float16
    np.testing.assert_allclose(out.float().numpy(), want, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("cuts", [(1,), (2, 5), (1, 2, 3, 4, 5, 6)])
def test_chunk_merge_equals_one_pass(cuts):
    # attention over 7 blocks computed in chunks of blocks by the oracle, then
    # merged pairwise: equal to one pass over all of them
    rng = np.random.default_rng(len(cuts))
    k = rng.standard_normal((7 * 8, 2, 32)).astype(np.float32)
    v = rng.standard_normal((7 * 8, 2, 32)).astype(np.float32)
    q = rng.standard_normal((4, 32)).astype(np.float32)
    pk, sk, valid = O.quantize_blocks(k, 4, 16, 8)
    pv, sv, _ = O.quantize_blocks(v, 4, 16, 8)
    valid[3] = 2
    full, full_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 16, 0.2)
    edges = [0, *cuts, 7]
    acc = None
    for a, b in zip(edges, edges[1:]):
        o, lse = O.attention(q, pk[a:b], pv[a:b], sk[a:b], sv[a:b], valid[a:b], 4, 16, 0.2)
        part = (torch.from_numpy(o), torch.from_numpy(lse))
        acc = part if acc is None else merge_attention_chunks(*acc, *part)
    np.testing.assert_allclose(acc[0].numpy(), full, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(acc[1].numpy(), full_lse, rtol=1e-6, atol=1e-6)


def test_merge_with_an_empty_chunk_is_the_identity():
    out = torch.randn(4, 8)
    lse = torch.randn(4)
    empty_o, empty_l = torch.full((4, 8), float("nan")), torch.full((4,), float("-inf"))
    m, ml = merge_attention_chunks(out, lse, empty_o, empty_l)
    torch.testing.assert_close(m, out)
    torch.testing.assert_close(ml, lse)
    m, ml = merge_attention_chunks(empty_o, empty_l, empty_o, empty_l)
    assert torch.all(m == 0) and torch.all(torch.isneginf(ml))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh", "d"), [(1, 1, 32), (4, 1, 64), (4, 2, 128)])
def test_reference_backend_matches_oracle(bits: int, qh: int, kvh: int, d: int) -> None:
    gen = torch.Generator().manual_seed(41)
    query = torch.randn(qh, d, generator=gen)
    keys = torch.randn(2, 8, kvh, d, generator=gen)
    values = torch.randn(2, 8, kvh, d, generator=gen)
    kq, vq = quantize_tensor(keys, bits, 16), quantize_tensor(values, bits, 16)
    valid = torch.tensor([8, 5], dtype=torch.int32)
    batch = PackedBatch(kq.packed, vq.packed, kq.scales, vq.scales, valid, bits, 16)
    scale = 1 / math.sqrt(d)
    out, lse = ReferenceAttentionBackend().run(query, batch, scale)
    o_out, o_lse = O.attention(
        query.numpy(), kq.packed.numpy(), vq.packed.numpy(), kq.scales.numpy(), vq.scales.numpy(), valid.numpy(), bits, 16, scale
    )
    np.testing.assert_allclose(out.numpy(), o_out, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(lse.numpy(), o_lse, atol=2e-5, rtol=2e-5)


def test_reference_backend_negative_counts_slice_like_python():
    # valid = -3 keeps rows [:-3] of its block, valid = -40 keeps none
    gen = torch.Generator().manual_seed(8)
    query = torch.randn(2, 32, generator=gen)
    keys, values = torch.randn(3, 8, 1, 32, generator=gen), torch.randn(3, 8, 1, 32, generator=gen)
    kq, vq = quantize_tensor(keys, 4, 16), quantize_tensor(values, 4, 16)
    batch = PackedBatch(kq.packed, vq.packed, kq.scales, vq.scales, torch.tensor([-3, 8, -40], dtype=torch.int32), 4, 16)
    out, lse = ReferenceAttentionBackend().run(query, batch, 0.2)
    same = PackedBatch(kq.packed, vq.packed, kq.scales, vq.scales, torch.tensor([5, 8, 0], dtype=torch.int32), 4, 16)
    out2, lse2 = ReferenceAttentionBackend().run(query, same, 0.2)
    assert torch.equal(out, out2) and torch.equal(lse, lse2)
