"""Seeded sweep of vLLM block records for the GPU codec.

Each case draws the bit width, a pack-aligned group size, the number of groups
(from one group to ~1M values, so that small records, odd-sized payloads and
records spread over many workgroups all occur), the dtype and the value range.
The GPU encoder must write the oracle's ``KVVLLM02`` record byte for byte, and
the GPU decoder must turn that record into the oracle's values bit for bit in
the destination dtype.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvssd import vllm_codec_hip as V
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CODES = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
CASES = 60


def draw(seed: int):
    rng = np.random.default_rng(7000 + seed)
    bits = int(rng.choice([2, 4]))
    step = 8 // bits
    g = int(rng.choice([step, 2 * step, 8, 16, 32, 32, 64, 128, 256]))
    g = g - g % step or step
    groups = int(rng.choice([1, 2, 3, int(rng.integers(1, 500)), int(rng.integers(500, 40000))]))
    dtype = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
    return bits, g, groups, dtype, float(rng.choice([1e-3, 1.0, 100.0]))


@pytest.mark.parametrize("seed", range(CASES))
def test_random_vllm_record_round_trip(cuda_device, seed):
    bits, g, groups, dtype, vscale = draw(seed)
    gen = torch.Generator().manual_seed(seed)
    x = (torch.randn(groups * g, generator=gen) * vscale).to(dtype)
    case = f"bits={bits} g={g} groups={groups} {dtype}"
    want = O.encode_vllm_record(x.float().numpy(), bits, g, CODES[dtype])
    rec = V.encode_vllm_block(x.to(cuda_device), bits=bits, group_size=g)
    assert rec.numel() == len(want), case
    assert rec.cpu().numpy().tobytes() == want, case

    dst = torch.full_like(x, 7.0, device=cuda_device)
    info = V.decode_vllm_block(rec, dst)
    assert (info.bits, info.group_size, info.dtype, info.elements) == (bits, g, dtype, x.numel()), case
    ref = torch.from_numpy(O.decode_vllm_values(want)).to(dtype)
    assert torch.equal(dst.cpu().view(torch.uint8), ref.view(torch.uint8)), case
