"""GPU parity of the staged kernel over the shapes that decide which blocks a
split attends: an INT4 split s takes units s, s + splits, s + 2 splits, ...
(an INT2 split a contiguous run), so unit counts that the split count does not
divide, split counts that are not a multiple of the 8 XCDs, the switch between
4 and 8 kv heads per workgroup around 2048 (kv head, block) pairs, block
tables with repeats, and empty blocks are each checked against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvssd.backends.hip import HipAttentionBackend
from oracle import oracle as O

from test_gpu_decode import ATOL, RTOL, make_batch, to_device

pytestmark = pytest.mark.gpu

# (kv heads, blocks, table): 257 and 300 blocks x 8 kv heads give 8 kv heads per
# workgroup with 2 blocks per split (129 / 150 splits); 520 x 8 gives 3 blocks
# per split (174 splits, the last round partial); 300 x 4 and 100 x 8 take 4 kv
# heads per workgroup (150 / 100 splits).
CASES = [
    (8, 257, None),
    (8, 300, None),
    (8, 520, None),
    (4, 300, None),
    (8, 100, None),
    (8, 300, "repeats"),
    (4, 300, "repeats"),
]


def _table(kind, nb, rng):
    if kind is None:
        return None
    # as many entries as blocks: a permutation with a tenth of the entries
    # replaced by repeats of others
    ids = rng.permutation(nb)
    ids[rng.random(nb) < 0.1] = rng.integers(0, nb)
    return ids.astype(np.int32)


@pytest.mark.parametrize("bits", [4, 2])
@pytest.mark.parametrize("gq", [4, 8])
@pytest.mark.parametrize(("kvh", "nb", "table"), CASES)
def test_staged_split_shapes(cuda_device, bits, gq, kvh, nb, table):
    rng = np.random.default_rng(nb * 31 + kvh * 7 + bits + gq)
    valid = rng.integers(1, 129, nb)
    valid[rng.random(nb) < 0.05] = 0  # empty blocks: their stages are skipped
    q, pk, pv, sk, sv, valid = make_batch(nb + kvh, gq * kvh, kvh, 128, nb, 128, bits, 32, valid=valid)
    ids = _table(table, nb, rng)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, torch.float16)
    backend = HipAttentionBackend("staged")
    assert backend.kernel_for(query, batch) == "staged"
    out, lse = backend.run(query, batch, 0.088, block_table=None if ids is None else torch.from_numpy(ids))
    torch.cuda.synchronize()
    ref_out, ref_lse = O.attention(
        query.float().cpu().numpy(), pk, pv, sk, sv, valid, bits, 32, 0.088, block_table=ids, threads=16
    )
    got = out.cpu().numpy()
    np.testing.assert_allclose(got, ref_out, atol=ATOL, rtol=RTOL)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL)
    # norm-relative: an all-zero or half-missing output cannot pass
    assert np.linalg.norm(got - ref_out) <= 1e-2 * np.linalg.norm(ref_out)
    assert np.max(np.abs(lse.cpu().numpy() - ref_lse)) <= 2e-3
    # control: the same checks see one unit fewer (the last one, which falls in
    # the last, partial round of the interleaved order) -- the fullest block
    # there is swapped in, so the missing share is large enough to show
    units = np.arange(nb, dtype=np.int32) if ids is None else ids
    last = units.copy()
    last[-1] = units[int(np.argmax(valid[units]))]
    ref_last, lse_last = O.attention(
        query.float().cpu().numpy(), pk, pv, sk, sv, valid, bits, 32, 0.088, block_table=last, threads=16
    )
    fewer, lse_fewer = O.attention(
        query.float().cpu().numpy(), pk, pv, sk, sv, valid, bits, 32, 0.088, block_table=last[:-1], threads=16
    )
    assert np.max(np.abs(lse_last - lse_fewer)) > 2e-3
