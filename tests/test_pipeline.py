"""Pipeline on CPU: the reference's test (tests/test_pipeline.py:11-23) plus
equality with the oracle over the selected blocks."""

import math
from pathlib import Path

import numpy as np
import torch

from kvssd.format import CacheSpec
from kvssd.pipeline import KVSSDPipeline
from kvssd.selectors import RecentSinkBlocks
from kvssd.store import KVCacheStore
from oracle import oracle as O


def test_cpu_end_to_end_with_selection(tmp_path: Path) -> None:
    gen = torch.Generator().manual_seed(11)
    shape = (1, 40, 2, 32)
    keys, values = torch.randn(shape, generator=gen), torch.randn(shape, generator=gen)
    store = KVCacheStore.create(tmp_path, keys, values, CacheSpec(1, 2, 32, block_tokens=8, bits=4, group_size=16))
    query = torch.randn(4, 32, generator=gen)
    with KVSSDPipeline(store, device="cpu", io_depth=2) as pipeline:
        output = pipeline.decode(query, 0, RecentSinkBlocks(1, 2))
    assert output.shape == (4, 32)
    assert torch.isfinite(output).all()
    pk, sk, valid = O.quantize_blocks(keys[0].numpy(), 4, 16, 8)
    pv, sv, _ = O.quantize_blocks(values[0].numpy(), 4, 16, 8)
    table = np.array(O.select_recent_sink(list(range(5)), 1, 2), np.int32)
    expect, _ = O.attention(query.numpy(), pk, pv, sk, sv, valid, 4, 16, 1 / math.sqrt(32), block_table=table)
    np.testing.assert_allclose(output.numpy(), expect, atol=2e-5, rtol=2e-5)
