"""GPU vLLM block codec against the oracle (tests/test_oracle.py pins the
oracle's record to a hand-assembled known answer and zlib).

Bars: record bytes bit-exact; decoded values bit-exact in the destination
dtype ((code - mid) * scale in fp32, one rounding, as dequantize_tensor)."""

from __future__ import annotations

import struct

import numpy as np
import pytest
import torch

from kvssd import vllm_codec_hip as V
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CODES = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
CASES = [
    # (shape, bits, group_size): one row; 41 rows behind 8,192 virtual zero
    # bytes; a 3-byte payload (byte path); group 16 and 64
    ((16, 8, 128), 4, 32),
    ((2, 16, 8, 128), 2, 32),
    ((9, 16, 8, 128, 8), 4, 32),
    ((4,), 2, 4),
    ((3, 5, 64), 4, 16),
    ((7, 64), 2, 64),
]


def values(shape, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=gen) * 2
    x.view(-1)[:: max(1, x.numel() // 7)] *= 8  # a few outliers
    return x.to(dtype)


def expected(x: torch.Tensor, bits: int, g: int) -> bytes:
    return O.encode_vllm_record(x.float().numpy(), bits, g, CODES[x.dtype])


@pytest.mark.parametrize(("shape", "bits", "g"), CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_encode_bit_exact(cuda_device, shape, bits, g, dtype):
    x = values(shape, dtype, 3 + bits + g)
    rec = V.encode_vllm_block(x.to(cuda_device), bits=bits, group_size=g)
    want = expected(x, bits, g)
    assert rec.numel() == len(want)
    assert rec.cpu().numpy().tobytes() == want


@pytest.mark.parametrize(("shape", "bits", "g"), CASES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("where", ["host", "device"])
def test_decode_bit_exact(cuda_device, shape, bits, g, dtype, where):
    x = values(shape, dtype, 5 + bits)
    rec = torch.from_numpy(np.frombuffer(expected(x, bits, g), dtype=np.uint8).copy())
    if where == "device":
        rec = rec.to(cuda_device)
    dst = torch.full(shape, 123.0, dtype=dtype, device=cuda_device)
    info = V.decode_vllm_block(rec, dst)
    assert (info.bits, info.group_size, info.dtype, info.elements) == (bits, g, dtype, x.numel())
    want = torch.from_numpy(O.decode_vllm_values(rec.cpu().numpy().tobytes())).to(dtype).reshape(shape)
    assert torch.equal(dst.cpu().view(torch.uint8), want.view(torch.uint8))


def test_round_trip_on_device(cuda_device):
    x = values((8, 16, 8, 128), torch.bfloat16, 1).to(cuda_device)
    rec = V.encode_vllm_block(x, bits=4, group_size=32)
    out = torch.empty_like(x)
    V.decode_vllm_block(rec, out)
    step = x.float().view(-1, 32).abs().amax(1, keepdim=True) / 7
    err = (out.float() - x.float()).view(-1, 32).abs()
    assert bool((err <= 0.51 * step + 0.01 * step.clamp_min(1e-3)).all())


def corrupt(rec: bytes, at: int, value: bytes) -> torch.Tensor:
    b = bytearray(rec)
    b[at : at + len(value)] = value
    return torch.from_numpy(np.frombuffer(bytes(b), dtype=np.uint8).copy())


def test_decode_errors_match_the_reference(cuda_device):
    x = values((16, 8, 128), torch.float16, 2)
    rec = expected(x, 4, 32)
    dst = torch.empty((16, 8, 128), dtype=torch.float16, device=cuda_device)
    plen = struct.unpack_from("<8sBBBBIIQI", rec)[7]
    with pytest.raises(ValueError, match="truncated KVSSD vLLM record"):
        V.decode_vllm_block(torch.zeros(10, dtype=torch.uint8), dst)
    with pytest.raises(ValueError, match="invalid KVSSD vLLM record header"):
        V.decode_vllm_block(corrupt(rec, 0, b"KVVLLM01"), dst)
    with pytest.raises(ValueError, match="invalid KVSSD vLLM record header"):
        V.decode_vllm_block(corrupt(rec, 8, b"\x02"), dst)
    with pytest.raises(ValueError, match="unsupported KVSSD vLLM dtype code 9"):
        V.decode_vllm_block(corrupt(rec, 10, b"\x09"), dst)
    with pytest.raises(ValueError, match="truncated KVSSD vLLM payload"):
        V.decode_vllm_block(torch.from_numpy(np.frombuffer(rec[: 32 + plen - 1], dtype=np.uint8).copy()), dst)
    with pytest.raises(IOError, match="CRC mismatch"):
        V.decode_vllm_block(corrupt(rec, 32 + 5000, b"\x00\x00"), dst)
    with pytest.raises(IOError, match="CRC mismatch"):  # GPU path, device record
        V.decode_vllm_block(corrupt(rec, 32 + plen - 1, b"\x77").to(cuda_device), dst)
    with pytest.raises(ValueError, match="destination has 8192 values, record requires 16384"):
        V.decode_vllm_block(torch.from_numpy(np.frombuffer(rec, dtype=np.uint8).copy()), dst[:8])
    with pytest.raises(ValueError, match="not divisible"):
        V.decode_vllm_block(torch.from_numpy(np.frombuffer(rec, dtype=np.uint8).copy()), dst.view(torch.uint8).view(-1)[:-1])
    # a layout that does not add up, CRC intact: ValueError; CRC broken too: IOError first
    bad = struct.pack("<I", 16000)
    with pytest.raises(ValueError, match="layout is inconsistent"):
        V.decode_vllm_block(corrupt(rec, 16, bad), dst)
    with pytest.raises(IOError, match="CRC mismatch"):
        V.decode_vllm_block(corrupt(bytes(corrupt(rec, 16, bad).numpy()), 40, b"\x01"), dst)


def test_encode_rejects_what_the_reference_rejects(cuda_device):
    with pytest.raises(ValueError, match="not divisible by group_size=32"):
        V.encode_vllm_block(torch.zeros(40, device=cuda_device), bits=4, group_size=32)
    with pytest.raises(KeyError):
        V.encode_vllm_block(torch.zeros(64, dtype=torch.float64, device=cuda_device), bits=4, group_size=32)
    with pytest.raises(ValueError):
        V.encode_vllm_block(torch.zeros(64, device=cuda_device), bits=3, group_size=32)
