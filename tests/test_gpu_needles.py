"""Full-size parity that can see missing work: needle tokens (tests/needles.py)
in every 32-token segment of every attended block, a check of out and lse
tight enough to notice one dropped needle, segment or block, and negative
controls proving it: each kernel's result must FAIL the same check against
the oracle over the selection with one block, one 32-token segment or one
needle removed.

Workloads: INT4 GQA 4 at 131,072 tokens (values x0.5), INT2 at 131,072 tokens
(5% x8 outliers), INT4 GQA 8 at 262,144 tokens through RecentSinkBlocks(1, 32),
the 1,048,576-token host-staged stream, and the 8-kv-head-per-workgroup shapes
with empty and partial blocks at split starts and a scattered block table.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import needles as N
from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend
from kvssd.format import CacheSpec
from kvssd.selectors import RecentSinkBlocks

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)
KERNELS = ("general", "mfma", "staged")


def run_kernels(dev, q16, arrays, valid, bits, table=None, kernels=KERNELS):
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in arrays), torch.from_numpy(valid).to(dev), bits, 32)
    results = {}
    for kernel in kernels:
        out, lse = HipAttentionBackend(kernel).run(q16.to(dev), batch, SCALE, block_table=table)
        results[kernel] = (out.cpu().numpy(), lse.cpu().numpy())
    return results


def check_case(dev, q16, arrays, valid, bits, table, needles, kernels=KERNELS, single_needle=True, what=""):
    q = q16.float().numpy()
    ref_out, ref_lse = N.oracle(q, arrays, valid, bits, table)
    share = N.needle_mass_share(q, arrays[0], arrays[2], bits, needles, ref_lse)
    assert share > 0.98, f"needles carry only {share:.3f} of the mass"
    results = run_kernels(dev, q16, arrays, valid, bits, table, kernels)
    for kernel, (out, lse) in results.items():
        N.assert_sensitive_match(out, lse, ref_out, ref_lse, f"{what} {kernel}")
    for name, (c_out, c_lse) in N.controls(q, arrays, valid, bits, table, needles, single_needle).items():
        for kernel, (out, lse) in results.items():
            assert N.differs(out, lse, c_out, c_lse), f"{what} {kernel}: the check would pass with one {name} dropped"


@pytest.mark.parametrize(("bits", "value_scale", "outliers", "target"), [(4, 0.5, 0.0, 10.0), (2, 1.0, 0.05, 16.0)])
def test_needles_128k_tokens(cuda_device, bits, value_scale, outliers, target):
    q16, k, v = N.half_kv(131072, 7, value_scale, outliers, 32)
    rng = np.random.default_rng(100 + bits)
    valid = np.full(1024, 128, np.int32)
    needles = N.plant(k.reshape(1024, 128, 8, 128), v.reshape(1024, 128, 8, 128), q16.float().numpy(), valid,
                      SCALE, rng, amp=512.0, target=target)
    arrays, valid = N.quantize(k, v, bits)
    del k, v
    check_case(cuda_device, q16, arrays, valid, bits, None, needles, what=f"INT{bits} 128K")


def test_needles_sparse_262k_tokens_gqa8(cuda_device):
    q16, k, v = N.half_kv(262144, 11, 1.0, 0.0, 64)
    ids = RecentSinkBlocks(1, 32).select(list(range(2048)))
    rng = np.random.default_rng(262)
    valid = np.full(2048, 128, np.int32)
    needles = N.plant(k.reshape(2048, 128, 8, 128), v.reshape(2048, 128, 8, 128), q16.float().numpy(), valid,
                      SCALE, rng, amp=64.0, blocks=ids)
    arrays, valid = N.quantize(k, v, 4)
    del k, v
    check_case(cuda_device, q16, arrays, valid, 4, ids, needles, what="sparse 262K GQA 8")


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh"), [(32, 8), (64, 8), (48, 16)])
def test_needles_eight_kv_heads_per_workgroup(cuda_device, bits, qh, kvh):
    # the staged kernel's 8-kv-head layout, empty and partial blocks at split
    # starts, then the same blocks through a scattered table
    rng = np.random.default_rng(3000 + 100 * bits + qh + kvh)
    nb = 2048 // kvh + 64
    q16, k, v = N.half_kv(nb * 128, 5 + qh + kvh, 1.0, 0.0, qh, kvh)
    valid = rng.integers(1, 129, nb).astype(np.int32)
    valid[::4] = 0
    valid[1::8] = rng.integers(0, 3, nb // 8)
    valid[2::16] = rng.integers(60, 70, nb // 16)
    valid[3::2] = 128
    needles = N.plant(k.reshape(nb, 128, kvh, 128), v.reshape(nb, 128, kvh, 128), q16.float().numpy(), valid,
                      SCALE, rng, amp=64.0, target=12.0)
    arrays, _ = N.quantize(k, v, bits)
    del k, v
    check_case(cuda_device, q16, arrays, valid, bits, None, needles, kernels=("staged",), what="8 kv heads")
    ids = [int(i) for i in rng.permutation(nb)[: 2048 // kvh + 40]]
    sel = set(ids)
    keep = np.isin(needles[0], list(sel))
    check_case(cuda_device, q16, arrays, valid, bits, ids, (needles[0][keep], needles[1][keep]),
               kernels=("staged",), what="8 kv heads, table")


def test_needles_host_staged_1m_tokens(cuda_device):
    # the 1,048,576-token host-staged stream: needles planted in the device
    # K/V before the records are encoded.  With 131,072 needles per kv head one
    # needle moves the output by less than the tolerance, so the four needles
    # of a segment share their dim and sign (a dropped segment moves one dim by
    # 4 amp / N) and the controls are one block and one 32-token segment
    from kvssd import records_hip as R
    from kvssd.staging import HostRecords, RecordStager

    spec = CacheSpec(1, 8, 128, 128, 4, 32)
    nb, dev = 8192, cuda_device
    gen = torch.Generator(device=dev).manual_seed(17)
    keys = torch.randn(nb * 128, 8, 128, generator=gen, device=dev, dtype=torch.float16)
    values = torch.randn(nb * 128, 8, 128, generator=gen, device=dev, dtype=torch.float16)
    q16 = torch.randn(32, 128, generator=gen, device=dev, dtype=torch.float16).cpu()
    rng = np.random.default_rng(1048576)
    valid = np.full(nb, 128, np.int32)
    bb, tt = N.needle_rows(valid, 128, rng)
    rows = torch.from_numpy(bb * 128 + tt).to(dev)
    nk = torch.from_numpy(N.needle_keys(q16.float().numpy(), 8, SCALE)).to(dev).half()
    keys[rows] = nk[None].expand(len(bb), 8, 128)
    values[rows] = torch.from_numpy(N.needle_values(len(bb), 8, 128, 1024.0, rng, run=4)).to(dev).half()
    records, _ = R.encode_records(keys, values, spec, layer=0)
    del keys, values
    pinned = torch.empty(records.shape, dtype=torch.uint8, pin_memory=True)
    pinned.copy_(records)
    del records
    backend = HipAttentionBackend()
    stager = RecordStager(spec, dev, 64, backend, torch.cuda.Stream(dev), torch.cuda.Stream(dev))
    ids = list(range(nb))
    out, lse = stager.run(q16.to(dev), SCALE, 0, ids, stager.host_fill(HostRecords(pinned, ids)))
    torch.cuda.synchronize()
    out, lse = out.cpu().numpy(), lse.cpu().numpy()

    raw = pinned.numpy()
    s, pb, base = 128 * 8 * 4 * 2, 128 * 8 * 64, 52
    sk = np.ascontiguousarray(raw[:, base : base + s]).view(np.float16).reshape(nb, 128, 8, 4)
    sv = np.ascontiguousarray(raw[:, base + s : base + 2 * s]).view(np.float16).reshape(nb, 128, 8, 4)
    pk = np.ascontiguousarray(raw[:, base + 2 * s : base + 2 * s + pb]).reshape(nb, 128, 8, 64)
    pv = np.ascontiguousarray(raw[:, base + 2 * s + pb : base + 2 * s + 2 * pb]).reshape(nb, 128, 8, 64)
    arrays = [pk, pv, sk, sv]
    q = q16.float().numpy()
    ref_out, ref_lse = N.oracle(q, arrays, valid, 4)
    assert N.needle_mass_share(q, pk, sk, 4, (bb, tt), ref_lse) > 0.98
    N.assert_sensitive_match(out, lse, ref_out, ref_lse, "host-staged 1M")
    for name, (c_out, c_lse) in N.controls(q, arrays, valid, 4, None, (bb, tt), single_needle=False).items():
        assert N.differs(out, lse, c_out, c_lse), f"the check would pass with one {name} dropped"
