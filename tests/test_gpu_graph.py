"""HIP graph capture of the fused decode.

A serving loop captures its decode step once and replays it.  The HIP backend
launches its kernels on torch's current stream and neither synchronises,
allocates through the runtime nor clears memory, so the captured launches
replay the same decode.  Every replay is checked bit for bit against an eager
call on the same inputs, with the program's own eager work (a new query copied
in place) between replays, and the first against the CPU oracle.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def _batch(dev, seed: int, qh: int, nb: int, bits: int, kvh: int = 8, d: int = 128, bt: int = 128, g: int = 32):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    v = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    pk, sk, _ = O.quantize_blocks(k, bits, g, bt)
    pv, sv, _ = O.quantize_blocks(v, bits, g, bt)
    valid = rng.integers(1, bt + 1, nb).astype(np.int32)
    host = (pk, pv, sk, sv, valid)
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in host), bits, g)
    queries = [rng.standard_normal((qh, d)).astype(np.float32) for _ in range(4)]
    return host, batch, queries


@pytest.mark.parametrize(
    "bits,qh,nb,table",
    [(4, 32, 1024, None), (2, 32, 96, None), (4, 64, 64, "recent"), (4, 32, 40, None)],
    ids=["int4-128k", "int2", "int4-gqa8-table", "int4-small"],
)
def test_fused_decode_replays_in_a_graph(cuda_device, bits, qh, nb, table):
    host, batch, queries = _batch(cuda_device, 40 + nb, qh, nb, bits)
    backend = HipAttentionBackend()
    scale = 1 / math.sqrt(128)
    ids = None
    if table is not None:
        ids = np.array([0] + list(range(nb - 16, nb)), np.int32)
    dtab = None if ids is None else torch.from_numpy(ids).to(cuda_device)
    query = torch.from_numpy(queries[0]).to(torch.float16).to(cuda_device)

    side = torch.cuda.Stream(cuda_device)
    side.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(side):
        backend.run(query, batch, scale, block_table=dtab)  # warm the shape's plan off the capture
    torch.cuda.current_stream(cuda_device).wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, g_lse = backend.run(query, batch, scale, block_table=dtab)

    for r, qn in enumerate(queries):
        query.copy_(torch.from_numpy(qn).to(torch.float16).to(cuda_device))
        graph.replay()
        e_out, e_lse = backend.run(query, batch, scale, block_table=dtab)
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out), f"replay {r}: out differs from the eager decode"
        assert torch.equal(g_lse, e_lse), f"replay {r}: lse differs from the eager decode"
        if r == 0:
            q = query.float().cpu().numpy()
            ref_out, ref_lse = O.attention(q, *host, bits, 32, scale, block_table=ids)
            np.testing.assert_allclose(g_out.cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL)
            np.testing.assert_allclose(g_lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL)
    del graph
