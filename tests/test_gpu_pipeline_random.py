"""Seeded sweep of stores through every decode route of the pipeline.

Each case draws a store layout (layers, kv heads, head dim, block size, bits,
group size), a token count, the query heads and dtype, the staging chunk size
and a selector, builds the store (on the host or on the GPU, alternately), and
decodes one layer three ways: streamed from the SSD, from page-locked host
records, and from HBM-resident blocks.  Each result is checked against the CPU
oracle over the same quantised blocks at the contract tolerance.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd import KVCacheStore, KVSSDPipeline
from kvssd.format import CacheSpec
from kvssd.selectors import AllBlocks, RecentSinkBlocks
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
CASES = 40


def draw(seed: int):
    rng = np.random.default_rng(9000 + seed)
    bits = int(rng.choice([2, 4]))
    kvh = int(rng.choice([1, 2, 4, 8]))
    d = int(rng.choice([64, 128, 128]))
    g = int(rng.choice([16, 32, 32, 64]))
    bt = int(rng.choice([16, 64, 128, 128]))
    layers = int(rng.choice([1, 2]))
    tokens = int(rng.integers(1, 40 * bt // 4 + 2))
    gq = int(rng.choice([1, 2, 4, 8]))
    stage = int(rng.choice([1, 2, 5, 64]))
    n = -(-tokens // bt)
    kind = int(rng.integers(0, 3))
    if kind == 0:
        selector = AllBlocks()
    else:
        selector = RecentSinkBlocks(int(rng.integers(0, 3)), int(rng.integers(0 if kind == 2 else 1, n + 2)))
    qdtype = torch.float16 if rng.random() < 0.7 else torch.float32
    return CacheSpec(layers, kvh, d, bt, bits, g), tokens, kvh * gq, stage, selector, qdtype, bool(seed % 2)


@pytest.mark.parametrize("seed", range(CASES))
def test_random_store_every_route(cuda_device, tmp_path: Path, seed):
    spec, tokens, qh, stage, selector, qdtype, on_gpu = draw(seed)
    gen = torch.Generator().manual_seed(seed)
    shape = (spec.layers, tokens, spec.kv_heads, spec.head_dim)
    keys = torch.randn(shape, generator=gen, dtype=torch.float16)
    values = torch.randn(shape, generator=gen, dtype=torch.float16)
    if on_gpu:
        store = KVCacheStore.create(tmp_path, keys.to(cuda_device), values.to(cuda_device), spec)
    else:
        store = KVCacheStore.create(tmp_path, keys, values, spec)
    layer = spec.layers - 1
    query = torch.randn(qh, spec.head_dim, generator=gen, dtype=torch.float32).to(qdtype)
    n = -(-tokens // spec.block_tokens)
    ids = selector.select(list(range(n)))
    case = f"{spec} tokens={tokens} qh={qh} stage={stage} {selector} gpu_store={on_gpu}"
    if not ids:
        return  # the pipeline raises for an empty selection (tested elsewhere)
    pk, sk, valid = O.quantize_blocks(keys[layer].float().numpy(), spec.bits, spec.group_size, spec.block_tokens)
    pv, sv, _ = O.quantize_blocks(values[layer].float().numpy(), spec.bits, spec.group_size, spec.block_tokens)
    q = query.float().numpy()
    ref, _ = O.attention(
        q, pk, pv, sk, sv, valid, spec.bits, spec.group_size, 1 / math.sqrt(spec.head_dim),
        block_table=np.array(ids, np.int32),
    )
    with store, KVSSDPipeline(store, device=cuda_device, stage_blocks=stage, attention_backend="hip") as pipe:
        outs = {"streamed": pipe.decode(query, layer, selector)}
        pipe.load_host_resident([layer])
        outs["host"] = pipe.decode(query, layer, selector)
        pipe.load_resident([layer])
        outs["hbm"] = pipe.decode(query, layer, selector)
    for route, out in outs.items():
        assert out.dtype == qdtype and out.shape == (qh, spec.head_dim), f"{route}: {case}"
        np.testing.assert_allclose(out.float().cpu().numpy(), ref, atol=ATOL, rtol=RTOL, err_msg=f"{route}: {case}")
