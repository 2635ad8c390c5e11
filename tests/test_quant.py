"""The INT2/INT4 codec on the CPU: the error bound of the round trip, the
argument checks of src/kvssd/quant.py:17-25, bit-exact agreement with the
oracle's quantiser, and pack/unpack over every byte value."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvssd.quant import dequantize_tensor, pack_codes, quantize_tensor, unpack_codes
from oracle import oracle as O


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("group", [8, 32, 64])
def test_round_trip_error_is_at_most_half_a_step(bits, group):
    # inside the clamp range every value lands within half a quantisation step
    # of its code; the one clamped code (-mid, never produced) is out of play
    gen = torch.Generator().manual_seed(bits + group)
    x = torch.randn(5, 3, 128, generator=gen) * torch.rand(5, 3, 1, generator=gen) * 3
    q = quantize_tensor(x, bits, group)
    back = dequantize_tensor(q)
    assert back.shape == x.shape and back.dtype == torch.float32
    assert q.packed.shape == (5, 3, 128 * bits // 8) and q.scales.shape == (5, 3, 128 // group)
    step = q.scales.float().repeat_interleave(group, dim=-1)
    # fp16 rounding of the stored scale moves a code by at most pmax * 2^-11 steps
    slack = (2 ** (bits - 1) - 1) * 2.0**-11 * step + 1e-6
    assert torch.all((x - back).abs() <= step / 2 + slack)


@pytest.mark.parametrize(("bits", "mae_bound"), [(4, 0.12), (2, 0.65)])
def test_mean_error_on_unit_normal_data(bits, mae_bound):
    # the reference's published bounds for N(0, 1) values in groups of 32
    for seed in range(4):
        x = torch.randn(16, 8, 128, generator=torch.Generator().manual_seed(seed))
        err = (dequantize_tensor(quantize_tensor(x, bits, 32)) - x).abs().mean().item()
        assert err < mae_bound


def test_argument_checks():
    with pytest.raises(ValueError, match="divisible by group_size"):
        quantize_tensor(torch.randn(2, 31), 4, group_size=16)
    with pytest.raises(ValueError, match="bits must be 2 or 4"):
        quantize_tensor(torch.randn(2, 32), 3, group_size=16)
    with pytest.raises(ValueError, match="pack-aligned"):
        quantize_tensor(torch.randn(2, 32), 2, group_size=2)
    with pytest.raises(TypeError, match="floating point"):
        quantize_tensor(torch.ones(2, 32, dtype=torch.int32), 4, group_size=16)
    with pytest.raises(ValueError, match="byte aligned"):
        pack_codes(torch.zeros(3, dtype=torch.uint8), 2)


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
