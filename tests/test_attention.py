"""Attention orchestration on CPU: the reference's tests (tests/test_attention.py:11-64)
plus agreement of the portable backend with the oracle."""

from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.attention import merge_attention_chunks, packed_attention, reference_attention
from kvssd.backends import PackedBatch
from kvssd.backends.reference import ReferenceAttentionBackend
from kvssd.format import CacheSpec
from kvssd.quant import dequantize_tensor, quantize_tensor
from kvssd.store import KVCacheStore
from oracle import oracle as O


@pytest.mark.parametrize("bits", [2, 4])
def test_packed_attention_matches_dequantized_reference(tmp_path: Path, bits: int) -> None:
    gen = torch.Generator().manual_seed(5)
    keys = torch.randn(1, 13, 2, 32, generator=gen)
    values = torch.randn(1, 13, 2, 32, generator=gen)
    query = torch.randn(4, 32, generator=gen)
    spec = CacheSpec(1, 2, 32, block_tokens=8, bits=bits, group_size=16)
    store = KVCacheStore.create(tmp_path, keys, values, spec)
    blocks = [store.read(0, i) for i in store.blocks_for_layer(0)]
    actual = packed_attention(query, blocks)
    dequant_k = torch.cat([dequantize_tensor(x.key)[: x.valid_tokens] for x in blocks])
    dequant_v = torch.cat([dequantize_tensor(x.value)[: x.valid_tokens] for x in blocks])
    expected = reference_attention(query, dequant_k, dequant_v)
    torch.testing.assert_close(actual, expected)


def test_gqa_validation() -> None:
    with pytest.raises(ValueError, match="divisible"):
        reference_attention(torch.randn(3, 8), torch.randn(4, 2, 8), torch.randn(4, 2, 8))


def test_chunk_softmax_merge_matches_concatenation() -> None:
    gen = torch.Generator().manual_seed(17)
    query = torch.randn(4, 16, generator=gen)
    keys = torch.randn(11, 2, 16, generator=gen)
    values = torch.randn(11, 2, 16, generator=gen)
    mapping = torch.arange(4) // 2
    scores = torch.einsum("hd,thd->ht", query, keys[:, mapping]) / 4

    def chunk(start: int, end: int) -> tuple[torch.Tensor, torch.Tensor]:
        local = scores[:, start:end]
        lse = torch.logsumexp(local, dim=-1)
        out = torch.einsum("ht,thd->hd", torch.softmax(local, -1), values[start:end, mapping])
        return out, lse

    left, left_lse = chunk(0, 5)
    right, right_lse = chunk(5, 11)
    merged, _ = merge_attention_chunks(left, left_lse, right, right_lse)
    expected = reference_attention(query, keys, values)
    torch.testing.assert_close(merged, expected, atol=1e-6, rtol=1e-5)


def test_merge_with_empty_chunk_is_identity() -> None:
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
    scale = 1 / d**0.5
    out, lse = ReferenceAttentionBackend().run(query, batch, scale)
    o_out, o_lse = O.attention(
        query.numpy(), kq.packed.numpy(), vq.packed.numpy(), kq.scales.numpy(), vq.scales.numpy(), valid.numpy(), bits, 16, scale
    )
    np.testing.assert_allclose(out.numpy(), o_out, atol=2e-5, rtol=2e-5)
    np.testing.assert_allclose(lse.numpy(), o_lse, atol=2e-5, rtol=2e-5)
