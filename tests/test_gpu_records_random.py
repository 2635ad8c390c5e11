"""Seeded sweep of record layouts for the GPU record codec.

Each case draws a layout (bits, kv heads, head dim, group size, block size),
a token count (the last block usually partial), the source dtype, the value
range, the layer and the first block id.  The GPU encoder must write the
oracle's records byte for byte with their CRC-32 values, and the GPU gather
must turn the oracle's records back into the oracle's packed codes, fp16
scales and valid counts byte for byte.
"""

from __future__ import annotations

import zlib

import numpy as np
import pytest
import torch

from kvssd import records_hip as R
from kvssd.format import CacheSpec
from oracle import oracle as O

pytestmark = pytest.mark.gpu

CASES = 120


def draw(seed: int):
    rng = np.random.default_rng(5000 + seed)
    bits = int(rng.choice([2, 4]))
    kvh = int(rng.choice([1, 2, 3, 4, 8, 16]))
    d = int(rng.choice([4, 8, 16, 32, 64, 96, 128, 128, 256]))
    step = 8 // bits
    groups = [g for g in range(step, d + 1, step) if d % g == 0]
    g = int(rng.choice(groups))
    bt = int(rng.choice([1, 2, 3, 7, 16, 32, 48, 128, 256]))
    tokens = int(rng.integers(1, 5 * bt + 1))
    dtype = [torch.float16, torch.bfloat16, torch.float32][int(rng.integers(0, 3))]
    spec = CacheSpec(layers=1, kv_heads=kvh, head_dim=d, block_tokens=bt, bits=bits, group_size=g)
    return spec, tokens, dtype, float(rng.choice([0.01, 1.0, 50.0])), int(rng.integers(0, 80)), int(rng.integers(0, 1000))


def oracle_records(keys: np.ndarray, values: np.ndarray, spec: CacheSpec, layer: int, first_block: int) -> list[bytes]:
    pk, sk, valid = O.quantize_blocks(keys, spec.bits, spec.group_size, spec.block_tokens)
    pv, sv, _ = O.quantize_blocks(values, spec.bits, spec.group_size, spec.block_tokens)
    return [
        O.encode_record(
            layer, first_block + b, int(valid[b]), spec.bits, spec.block_tokens, spec.kv_heads, spec.head_dim,
            spec.group_size, sk[b], sv[b], pk[b], pv[b],
        )
        for b in range(pk.shape[0])
    ]


@pytest.mark.parametrize("seed", range(CASES))
def test_random_layout_encode_and_gather(cuda_device, seed):
    spec, tokens, dtype, vscale, layer, first = draw(seed)
    gen = torch.Generator().manual_seed(seed)
    k = (torch.randn(tokens, spec.kv_heads, spec.head_dim, generator=gen) * vscale).to(dtype)
    v = (torch.randn(tokens, spec.kv_heads, spec.head_dim, generator=gen) * vscale).to(dtype)
    want = oracle_records(k.float().numpy(), v.float().numpy(), spec, layer, first)
    case = f"{spec} tokens={tokens} {dtype}"

    recs, crcs = R.encode_records(k.to(cuda_device), v.to(cuda_device), spec, layer=layer, first_block=first)
    got = recs.cpu().numpy()
    assert got.shape == (len(want), spec.record_bytes), case
    for i, w in enumerate(want):
        assert got[i].tobytes() == w, f"record {i} differs: {case}"
        assert int(crcs[i]) == zlib.crc32(w[52 : 52 + int.from_bytes(w[44:48], "little")]), case

    raw = torch.from_numpy(np.frombuffer(b"".join(want), dtype=np.uint8).copy()).to(cuda_device)
    pk, pv, sk, sv, valid, status = R.gather_records(raw, spec, len(want))
    opk, osk, ovalid = O.quantize_blocks(k.float().numpy(), spec.bits, spec.group_size, spec.block_tokens)
    opv, osv, _ = O.quantize_blocks(v.float().numpy(), spec.bits, spec.group_size, spec.block_tokens)
    assert status.cpu().tolist() == [R.OK] * len(want), case
    assert np.array_equal(valid.cpu().numpy(), ovalid), case
    assert np.array_equal(pk.cpu().numpy(), opk), case
    assert np.array_equal(pv.cpu().numpy(), opv), case
    assert np.array_equal(sk.cpu().numpy().view(np.uint16), osk.view(np.uint16)), case
    assert np.array_equal(sv.cpu().numpy().view(np.uint16), osv.view(np.uint16)), case
