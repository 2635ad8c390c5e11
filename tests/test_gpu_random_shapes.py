"""Seeded sweep of decode shapes drawn from the whole supported domain.

Each case draws kv heads, GQA ratio, head dim, group size, block size, block
count, valid counts (including oversized ones, which keep the whole block, and
negative ones, which drop rows from the block's end as a Python slice does), an optional block table (any order, repeats allowed), the
query dtype, the softmax scale and the value range, and runs every kernel that
supports the shape against the CPU oracle at the contract tolerance
(max-abs 2e-3, rel 1e-2).  The draws are fixed by the seed, so a failure names
a reproducible case.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
CASES = 160


def draw(seed: int) -> dict:
    rng = np.random.default_rng(1000 + seed)
    bits = int(rng.choice([2, 4]))
    kvh = int(rng.choice([1, 2, 3, 4, 8, 12, 16]))
    gq = int(rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 10]))
    d = int(rng.choice([32, 64, 96, 128, 128, 128, 256]))
    groups = [g for g in (8, 16, 32, 64, 128) if d % g == 0 and g <= d]
    g = int(rng.choice(groups + [32] * 2 if d % 32 == 0 else groups))
    bt = int(rng.choice([8, 16, 32, 64, 128, 128, 256]))
    nb = int(rng.integers(1, 49))
    valid = rng.integers(-2, bt + 4, nb).astype(np.int32)
    if rng.random() < 0.5:
        valid[rng.random(nb) < 0.7] = bt  # mostly full blocks, as in a real cache
    table = None
    if rng.random() < 0.4:
        table = rng.integers(0, nb, int(rng.integers(1, nb + 6))).astype(np.int32)
    qdtype = [torch.float32, torch.float16, torch.bfloat16][int(rng.integers(0, 3))]
    return dict(
        bits=bits, kvh=kvh, qh=kvh * gq, d=d, g=g, bt=bt, nb=nb, valid=valid, table=table, qdtype=qdtype,
        scale=float(rng.uniform(0.05, 0.3)), vscale=float(rng.choice([0.25, 1.0, 3.0])), seed=seed,
    )


def kernels_for(query, batch):
    names = []
    for kernel in ("general", "mfma", "staged"):
        try:
            HipAttentionBackend(kernel).kernel_for(query, batch)
        except ValueError:
            continue
        names.append(kernel)
    return names


@pytest.mark.parametrize("seed", range(CASES))
def test_random_shape_matches_oracle(cuda_device, seed):
    c = draw(seed)
    rng = np.random.default_rng(seed)
    rows = c["nb"] * c["bt"]
    k = (rng.standard_normal((rows, c["kvh"], c["d"])) * c["vscale"]).astype(np.float32)
    v = (rng.standard_normal((rows, c["kvh"], c["d"])) * c["vscale"]).astype(np.float32)
    pk, sk, _ = O.quantize_blocks(k, c["bits"], c["g"], c["bt"])
    pv, sv, _ = O.quantize_blocks(v, c["bits"], c["g"], c["bt"])
    q = torch.from_numpy(rng.standard_normal((c["qh"], c["d"])).astype(np.float32)).to(c["qdtype"])
    qref = q.double().float().numpy()  # the values the kernel sees
    ref_out, ref_lse = O.attention(
        qref, pk, pv, sk, sv, c["valid"], c["bits"], c["g"], c["scale"], block_table=c["table"]
    )
    dev = cuda_device
    batch = PackedBatch(
        *(torch.from_numpy(a).to(dev) for a in (pk, pv, sk, sv, c["valid"])), c["bits"], c["g"]
    )
    query = q.to(dev)
    table = None if c["table"] is None else c["table"].tolist()
    kernels = kernels_for(query, batch)
    assert "general" in kernels
    desc = {key: c[key] for key in ("bits", "kvh", "qh", "d", "g", "bt", "nb", "qdtype")}
    for kernel in kernels:
        backend = HipAttentionBackend(kernel)
        out, lse = backend.run(query, batch, c["scale"], block_table=table)
        np.testing.assert_allclose(
            out.cpu().numpy(), ref_out, atol=ATOL, rtol=RTOL, err_msg=f"{kernel} {desc} table={table is not None}"
        )
        np.testing.assert_allclose(
            lse.cpu().numpy(), ref_lse, atol=ATOL, rtol=RTOL, err_msg=f"{kernel} {desc} table={table is not None}"
        )
