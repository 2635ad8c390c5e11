"""KVSSDPipeline.decode on the CPU: selection, bounded prefetch and the
portable backend, end to end against the oracle over the selected blocks
(the path of src/kvssd/pipeline.py:167-187 without a GPU)."""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.format import CacheSpec
from kvssd.pipeline import KVSSDPipeline
from kvssd.selectors import AllBlocks, RecentSinkBlocks
from kvssd.store import KVCacheStore
from oracle import oracle as O


@pytest.mark.parametrize("io_depth", [1, 2, 5])
def test_decode_over_selections_matches_the_oracle(tmp_path: Path, io_depth: int):
    gen = torch.Generator().manual_seed(70 + io_depth)
    keys = torch.randn(2, 75, 2, 32, generator=gen)  # 10 blocks of 8, the last holding 3 tokens
    values = torch.randn(2, 75, 2, 32, generator=gen)
    store = KVCacheStore.create(tmp_path, keys, values, CacheSpec(2, 2, 32, block_tokens=8, bits=4, group_size=16))
    query = torch.randn(4, 32, generator=gen, dtype=torch.float64)
    with KVSSDPipeline(store, device="cpu", io_depth=io_depth) as pipe:
        for layer in (0, 1):
            pk, sk, valid = O.quantize_blocks(keys[layer].numpy(), 4, 16, 8)
            pv, sv, _ = O.quantize_blocks(values[layer].numpy(), 4, 16, 8)
            for sel in (AllBlocks(), RecentSinkBlocks(1, 2), RecentSinkBlocks(0, 1), RecentSinkBlocks(3, 0)):
                out = pipe.decode(query, layer, sel)
                assert out.shape == (4, 32) and out.dtype == torch.float64
                ids = np.array(sel.select(list(range(10))), np.int32)
                expect, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 16, 1 / math.sqrt(32),
                                        block_table=ids)
                np.testing.assert_allclose(out.numpy(), expect, atol=2e-5, rtol=2e-5)
    store.close()


def test_resident_all_blocks_fast_path_selects_what_the_selector_would(tmp_path: Path):
    # A resident layer decoded under plain AllBlocks takes the batch's row order
    # as its selection without copying the id list; any other selector,
    # AllBlocks subclasses included, still goes through its own select().  The
    # layer is placed in the resident table on CPU tensors here, so the
    # portable backend serves the decode.
    from kvssd.backends import PackedBatch
    from kvssd.pipeline import _Resident

    gen = torch.Generator().manual_seed(91)
    keys = torch.randn(1, 75, 2, 32, generator=gen)
    values = torch.randn(1, 75, 2, 32, generator=gen)
    store = KVCacheStore.create(tmp_path, keys, values, CacheSpec(1, 2, 32, block_tokens=8, bits=4, group_size=16))
    query = torch.randn(4, 32, generator=gen, dtype=torch.float64)
    pk, sk, valid = O.quantize_blocks(keys[0].numpy(), 4, 16, 8)
    pv, sv, _ = O.quantize_blocks(values[0].numpy(), 4, 16, 8)
    ids = store.blocks_for_layer(0)
    assert ids == list(range(10))
    batch = PackedBatch(*(torch.from_numpy(a) for a in (pk, pv, sk, sv, valid)), 4, 16)

    class FirstTwo(AllBlocks):
        def select(self, available):
            return list(available)[:2]

    scale = 1 / math.sqrt(32)
    with KVSSDPipeline(store, device="cpu") as pipe:
        pipe._resident[0] = _Resident(batch, {b: i for i, b in enumerate(ids)}, list(ids))
        before = list(pipe._resident[0].ids)
        for sel, chosen in ((AllBlocks(), ids), (None, ids), (RecentSinkBlocks(0, 10), ids), (FirstTwo(), [0, 1])):
            out = pipe.decode(query, 0, sel)
            expect, _ = O.attention(query.float().numpy(), pk, pv, sk, sv, valid, 4, 16, scale,
                                    block_table=np.array(chosen, np.int32))
            np.testing.assert_allclose(out.numpy(), expect, atol=2e-5, rtol=2e-5)
        assert pipe._resident[0].ids == before
    store.close()
