"""Symmetric groupwise INT2/INT4 codec.

Semantics follow src/kvssd/quant.py:8-73 of the reference exactly, because the
packed bytes and fp16 scales produced here are the input of the fused HIP
kernel and must be bit-identical to what the reference writes:

* ``scale32 = max(|x|).clamp_min(1e-8) / (2^(bits-1) - 1)`` per group of
  ``group_size`` elements along the last dimension (quant.py:56);
* ``code = clamp(round_half_even(x / scale32), -mid, mid - 1) + mid``
  (quant.py:57-58), so codes are unsigned with midpoint ``mid = 2^(bits-1)``;
* codes are packed low bits first within each byte (quant.py:28-37);
* the stored scale is ``fp16(scale32)`` (quant.py:61) and dequantisation uses
  that fp16 value: ``(code - mid) * float(scale)`` (quant.py:68-73).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class QuantizedTensor:
    packed: torch.Tensor
    scales: torch.Tensor
    original_shape: tuple[int, ...]
    bits: int
    group_size: int


def _check(x: torch.Tensor, bits: int, group_size: int) -> None:
    # Error types and messages mirror src/kvssd/quant.py:17-25.
    if bits not in (2, 4):
        raise ValueError(f"bits must be 2 or 4, got {bits}")
    if group_size <= 0 or group_size % (8 // bits):
        raise ValueError("group_size must be positive and pack-aligned")
    if x.ndim < 1 or x.shape[-1] % group_size:
        raise ValueError("last dimension must be divisible by group_size")
    if not x.is_floating_point():
        raise TypeError("quantization input must be floating point")


def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Pack unsigned codes along the final dimension, low bits first."""
    if bits not in (2, 4):
        raise ValueError("bits must be 2 or 4")
    per_byte = 8 // bits
    if codes.shape[-1] % per_byte:
        raise ValueError("code dimension is not byte aligned")
    lanes = codes.to(torch.uint8).reshape(*codes.shape[:-1], -1, per_byte)
    mask = (1 << bits) - 1
    out = lanes[..., 0] & mask
    for slot in range(1, per_byte):
        out = out | ((lanes[..., slot] & mask) << (slot * bits))
    return out.to(torch.uint8).contiguous()


def unpack_codes(packed: torch.Tensor, bits: int, elements: int) -> torch.Tensor:
    """Unsigned codes from packed bytes; keeps the first ``elements`` codes."""
    if bits not in (2, 4):
        raise ValueError("bits must be 2 or 4")
    per_byte = 8 // bits
    mask = (1 << bits) - 1
    slots = [(packed >> (slot * bits)) & mask for slot in range(per_byte)]
    values = torch.stack(slots, dim=-1)
    return values.reshape(*packed.shape[:-1], -1)[..., :elements]


def quantize_tensor(x: torch.Tensor, bits: int, group_size: int = 32) -> QuantizedTensor:
    """Symmetric groupwise quantization suitable for register-level dequantization."""
    _check(x, bits, group_size)
    shape = tuple(x.shape)
    midpoint = 1 << (bits - 1)
    groups = x.float().reshape(*shape[:-1], shape[-1] // group_size, group_size)
    scale32 = groups.abs().amax(dim=-1).clamp_min(1e-8) / (midpoint - 1)
    rounded = torch.round(groups / scale32.unsqueeze(-1))
    codes = (rounded.clamp(-midpoint, midpoint - 1) + midpoint).to(torch.uint8).reshape(shape)
    return QuantizedTensor(
        packed=pack_codes(codes, bits),
        scales=scale32.to(torch.float16).contiguous(),
        original_shape=shape,
        bits=bits,
        group_size=group_size,
    )


def dequantize_tensor(q: QuantizedTensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    codes = unpack_codes(q.packed, q.bits, q.original_shape[-1]).to(torch.float32)
    midpoint = 1 << (q.bits - 1)
    groups = codes.reshape(*q.original_shape[:-1], -1, q.group_size) - midpoint
    values = groups * q.scales.float().unsqueeze(-1)
    return values.reshape(q.original_shape).to(dtype)
