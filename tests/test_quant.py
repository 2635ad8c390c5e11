"""Codec: the reference's tests (tests/test_quant.py:7-19) plus bit-exact
agreement with the oracle's quantiser and packer."""

import numpy as np
import pytest
import torch

from kvssd.quant import dequantize_tensor, pack_codes, quantize_tensor, unpack_codes
from oracle import oracle as O


@pytest.mark.parametrize(("bits", "max_mae"), [(4, 0.12), (2, 0.65)])
def test_quantization_round_trip(bits: int, max_mae: float) -> None:
    x = torch.randn(3, 2, 128, generator=torch.Generator().manual_seed(1))
    quantized = quantize_tensor(x, bits, group_size=32)
    restored = dequantize_tensor(quantized)
    assert restored.shape == x.shape
    assert torch.mean(torch.abs(x - restored)).item() < max_mae
    assert quantized.packed.numel() == x.numel() * bits // 8


def test_rejects_invalid_layout() -> None:
    with pytest.raises(ValueError, match="divisible"):
        quantize_tensor(torch.randn(2, 31), 4, group_size=16)
    with pytest.raises(ValueError, match="bits"):
        quantize_tensor(torch.randn(2, 32), 3, group_size=16)
    with pytest.raises(TypeError):
        quantize_tensor(torch.ones(2, 32, dtype=torch.int32), 4, group_size=16)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("group", [16, 32, 128])
def test_bit_exact_with_oracle(bits, dtype, group):
    gen = torch.Generator().manual_seed(bits * 100 + group)
    x = torch.randn(37, 8, 128, generator=gen) * torch.rand(37, 8, 1, generator=gen) * 4
    x[torch.rand(x.shape, generator=gen) < 0.05] *= 8
    x[3] = 0  # padding-like all-zero rows
    x = x.to(dtype)
    q = quantize_tensor(x, bits, group)
    codes, scales = O.quantize_c(x.float().numpy(), bits, group)
    assert np.array_equal(q.packed.numpy(), O.pack_np(codes, bits))
    assert np.array_equal(q.scales.view(torch.int16).numpy().view(np.uint16), scales.view(np.uint16))
    assert np.array_equal(unpack_codes(q.packed, bits, 128).numpy(), codes)
    deq = dequantize_tensor(q).numpy()
    assert np.array_equal(deq, O.dequantize_np(codes, scales, bits, group))


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_exhaustive(bits):
    every = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    codes = unpack_codes(every, bits, 256 * 8 // bits)
    assert np.array_equal(codes.numpy(), O.unpack_np(every.numpy(), bits))
    assert torch.equal(pack_codes(codes, bits), every)
