"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bars (from the path's contract):
  * unpacked integer codes and block selection: bit-exact;
  * dequantised values: exact (fp32);
  * attention out / lse: max-abs 2e-3, rel 1e-2 (fp32 accumulate), and the
    general kernel also at the reference's own GPU tolerance 2e-4
    (tests/test_triton_backend.py:110).
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from kvssd import _native
from kvssd.backends import PackedBatch, resolve_attention_backend
from kvssd.backends.hip import HipAttentionBackend
from oracle import oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2  # contract tolerance
REF_TOL = 2e-4  # reference GPU-test tolerance


def make_batch(seed, qh, kvh, d, nb, bt, bits, g, valid=None, value_scale=1.0, outliers=0.0):
    rng = np.random.default_rng(seed)
    k = (rng.standard_normal((nb * bt, kvh, d)) * value_scale).astype(np.float32)
    v = (rng.standard_normal((nb * bt, kvh, d)) * value_scale).astype(np.float32)
    if outliers:
        k[rng.random(k.shape) < outliers] *= 8
        v[rng.random(v.shape) < outliers] *= 8
    q = rng.standard_normal((qh, d)).astype(np.float32)
    pk, sk, _ = O.quantize_blocks(k, bits, g, bt)
    pv, sv, _ = O.quantize_blocks(v, bits, g, bt)
    if valid is None:
        valid = rng.integers(1, bt + 1, nb)
    return q, pk, pv, sk, sv, np.asarray(valid, np.int32)


def to_device(dev, q, pk, pv, sk, sv, valid, bits, g, qdtype=torch.float32):
    query = torch.from_numpy(q).to(qdtype).to(dev)
    batch = PackedBatch(
        torch.from_numpy(pk).to(dev),
        torch.from_numpy(pv).to(dev),
        torch.from_numpy(sk).to(dev),
        torch.from_numpy(sv).to(dev),
        torch.from_numpy(valid).to(dev),
        bits,
        g,
    )
    return query, batch


def check(out, lse, ref_out, ref_lse, atol=ATOL, rtol=RTOL):
    out, lse = out.cpu().numpy(), lse.cpu().numpy()
    np.testing.assert_allclose(out, ref_out, atol=atol, rtol=rtol)
    np.testing.assert_allclose(lse, ref_lse, atol=atol, rtol=rtol)


def kernels_for(query, batch):
    """Every kernel that supports this shape ("general" always)."""
    names = []
    for kernel in ("general", "mfma", "staged"):
        try:
            HipAttentionBackend(kernel).kernel_for(query, batch)
        except ValueError:
            continue
        names.append(kernel)
    return names


# ------------------------------------------------------------------ codec ---


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("n_bytes", [1, 3, 256, 4096 + 7, 1 << 20])
def test_unpack_codes_bit_exact(cuda_device, bits, n_bytes):
    rng = np.random.default_rng(n_bytes)
    packed = rng.integers(0, 256, n_bytes, dtype=np.uint8)
    packed[: min(256, n_bytes)] = np.arange(min(256, n_bytes), dtype=np.uint8)  # every byte value
    src = torch.from_numpy(packed).to(cuda_device)
    dst = torch.full((n_bytes * 8 // bits,), 255, dtype=torch.uint8, device=cuda_device)
    rc = _native.load().kvssd_hip_unpack_codes(src.data_ptr(), bits, n_bytes, dst.data_ptr(), None)
    _native.check(rc, "unpack")
    torch.cuda.synchronize()
    assert np.array_equal(dst.cpu().numpy(), O.unpack_np(packed, bits))


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("g", [16, 32, 128])
def test_dequantize_exact(cuda_device, bits, g):
    rng = np.random.default_rng(g + bits)
    x = (rng.standard_normal((300, 128)) * rng.choice([1e-4, 1.0, 100.0], (300, 1))).astype(np.float32)
    codes, scales = O.quantize_c(x, bits, g)
    packed = O.pack_np(codes, bits)
    out = torch.empty((300, 128), dtype=torch.float32, device=cuda_device)
    p = torch.from_numpy(packed).to(cuda_device)
    s = torch.from_numpy(scales.view(np.uint16).copy()).to(cuda_device)
    rc = _native.load().kvssd_hip_dequantize(p.data_ptr(), s.data_ptr(), 300, 128, bits, g, out.data_ptr(), None)
    _native.check(rc, "dequantize")
    assert np.array_equal(out.cpu().numpy(), O.dequantize_np(codes, scales, bits, g))


# ---------------------------------------------------------------- decode ---

MATRIX = [
    (1, 1, 32, 16, 32),
    (4, 1, 64, 16, 32),
    (4, 2, 128, 16, 32),
    (4, 2, 128, 32, 32),
    (1, 1, 128, 32, 128),
    (2, 1, 128, 32, 128),
    (4, 1, 128, 32, 128),
    (12, 2, 128, 32, 128),
    (32, 8, 128, 32, 128),
    (64, 8, 128, 32, 128),
    (32, 8, 128, 32, 256),
    (16, 4, 128, 32, 128),
    (8, 8, 128, 32, 128),
    (24, 12, 128, 32, 128),
    (40, 8, 128, 32, 128),
]


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh", "d", "g", "bt"), MATRIX)
def test_decode_matrix_fp32_query(cuda_device, bits, qh, kvh, d, g, bt):
    q, pk, pv, sk, sv, valid = make_batch(41, qh, kvh, d, 5, bt, bits, g)
    scale = 1 / math.sqrt(d)
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, bits, g, scale)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, g)
    for kernel in kernels_for(query, batch):
        backend = HipAttentionBackend(kernel)
        out, lse = backend.run(query, batch, scale)
        assert backend.last_kernel == kernel
        tol = REF_TOL if kernel == "general" else ATOL
        check(out, lse, ref_out, ref_lse, atol=tol, rtol=REF_TOL if kernel == "general" else RTOL)


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16, torch.float64])
@pytest.mark.parametrize("bits", [2, 4])
def test_decode_query_dtypes(cuda_device, qdtype, bits):
    q, pk, pv, sk, sv, valid = make_batch(7, 32, 8, 128, 4, 128, bits, 32)
    q = torch.from_numpy(q).to(qdtype).double().float().numpy()  # the values the kernel sees
    scale = 1 / math.sqrt(128)
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, bits, 32, scale)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype)
    assert "mfma" in kernels_for(query, batch)
    for kernel in kernels_for(query, batch):
        out, lse = HipAttentionBackend(kernel).run(query, batch, scale)
        check(out, lse, ref_out, ref_lse)


def test_decode_reference_test_shapes_block_tokens_8(cuda_device):
    # tests/test_triton_backend.py:13-31: 2 blocks x 8 tokens, valid [8, 5], g=16
    for bits in (2, 4):
        for qh, kvh, d in [(1, 1, 32), (4, 1, 64), (4, 2, 128)]:
            q, pk, pv, sk, sv, _ = make_batch(41, qh, kvh, d, 2, 8, bits, 16)
            valid = np.array([8, 5], np.int32)
            scale = 1 / math.sqrt(d)
            ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, bits, 16, scale)
            query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 16)
            out, lse = resolve_attention_backend("hip", cuda_device).run(query, batch, scale)
            check(out, lse, ref_out, ref_lse, atol=REF_TOL, rtol=REF_TOL)


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_edge_cases(cuda_device, bits):
    q, pk, pv, sk, sv, _ = make_batch(3, 32, 8, 128, 6, 256, bits, 32)
    scale = 0.1
    cases = {
        "zero_blocks": np.array([256, 0, 17, 0, 1, 129], np.int32),
        "oversize_and_negative": np.array([999, -4, 256, 3, 1000, 128], np.int32),
        "single_token": np.array([0, 0, 0, 1, 0, 0], np.int32),
        "sub_block_edges": np.array([127, 128, 129, 255, 16, 15], np.int32),
    }
    for name, valid in cases.items():
        ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, bits, 32, scale)
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32)
        for kernel in kernels_for(query, batch):
            out, lse = HipAttentionBackend(kernel).run(query, batch, scale)
            check(out, lse, ref_out, ref_lse)
    # no valid token at all: out = 0, lse = -inf (what the reference backend returns)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, np.zeros(6, np.int32), bits, 32)
    for kernel in kernels_for(query, batch):
        out, lse = HipAttentionBackend(kernel).run(query, batch, scale)
        assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


def test_decode_padding_garbage_is_ignored(cuda_device):
    q, pk, pv, sk, sv, valid = make_batch(4, 32, 8, 128, 3, 128, 4, 32, valid=[128, 10, 33])
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.1)
    rng = np.random.default_rng(0)
    for b, n in enumerate(valid):
        pk[b, n:] = rng.integers(0, 256, pk[b, n:].shape)
        pv[b, n:] = rng.integers(0, 256, pv[b, n:].shape)
        sk[b, n:] = np.float16(np.inf)
        sv[b, n:] = np.float16(np.nan)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32)
    for kernel in kernels_for(query, batch):
        out, lse = HipAttentionBackend(kernel).run(query, batch, 0.1)
        check(out, lse, ref_out, ref_lse)


@pytest.mark.parametrize("bits", [2, 4])
def test_block_table_selection(cuda_device, bits):
    q, pk, pv, sk, sv, valid = make_batch(8, 64, 8, 128, 40, 128, bits, 32)
    avail = list(range(40))
    for sink, recent in [(1, 32), (2, 3), (0, 1), (5, 0)]:
        ids = O.select_recent_sink(avail, sink, recent)
        table = np.array(ids, np.int32)
        ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, bits, 32, 0.09, block_table=table)
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32)
        for kernel in kernels_for(query, batch):
            out, lse = HipAttentionBackend(kernel).run(query, batch, 0.09, block_table=ids)
            check(out, lse, ref_out, ref_lse)
    with pytest.raises(ValueError, match="block ids"):
        HipAttentionBackend().run(query, batch, 0.09, block_table=[0, 40])


def test_config_cpu_runnable_4096_tokens(cuda_device):
    # 1 layer, 4096 tokens, KVH 8, QH 32, D 128, BT 128, INT4 g32, fp16 query
    gen = torch.Generator().manual_seed(7)
    k = torch.randn(4096, 8, 128, generator=gen, dtype=torch.float16)
    v = torch.randn(4096, 8, 128, generator=gen, dtype=torch.float16)
    q = torch.randn(32, 128, generator=gen, dtype=torch.float16)
    pk, sk, valid = O.quantize_blocks(k.float().numpy(), 4, 32, 128)
    pv, sv, _ = O.quantize_blocks(v.float().numpy(), 4, 32, 128)
    scale = 1 / math.sqrt(128)
    ref_out, ref_lse = O.attention(q.float().numpy(), pk, pv, sk, sv, valid, 4, 32, scale)
    query, batch = to_device(cuda_device, q.float().numpy(), pk, pv, sk, sv, valid, 4, 32, torch.float16)
    assert kernels_for(query, batch) == ["general", "mfma", "staged"]
    for kernel in kernels_for(query, batch):
        out, lse = HipAttentionBackend(kernel).run(query, batch, scale)
        check(out, lse, ref_out, ref_lse)


def test_merge_chunks_kernel(cuda_device):
    q, pk, pv, sk, sv, valid = make_batch(12, 32, 8, 128, 6, 32, 4, 32)
    halves = [slice(0, 2), slice(2, 6)]
    parts = [O.attention(q, pk[s], pv[s], sk[s], sv[s], valid[s], 4, 32, 0.1) for s in halves]
    full_out, full_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.1)
    acc_o = torch.from_numpy(parts[0][0]).to(cuda_device)
    acc_l = torch.from_numpy(parts[0][1]).to(cuda_device)
    HipAttentionBackend().merge_chunks(
        acc_o, acc_l, torch.from_numpy(parts[1][0]).to(cuda_device), torch.from_numpy(parts[1][1]).to(cuda_device)
    )
    check(acc_o, acc_l, full_out, full_lse, atol=1e-5, rtol=1e-5)
    empty_o = torch.full_like(acc_o, float("nan"))
    empty_l = torch.full_like(acc_l, float("-inf"))
    before = acc_o.clone()
    HipAttentionBackend().merge_chunks(acc_o, acc_l, empty_o, empty_l)
    torch.testing.assert_close(acc_o, before)


def test_library_shares_torch_hip_runtime(cuda_device):
    HipAttentionBackend().probe(cuda_device)
    maps = open("/proc/self/maps").read()
    paths = {line.split()[-1] for line in maps.splitlines() if "libamdhip64" in line}
    assert len(paths) == 1, paths
    assert any("libkvssd_hip.so" in line for line in maps.splitlines())


def test_misaligned_buffers_use_general_kernel(cuda_device):
    q, pk, pv, sk, sv, valid = make_batch(5, 32, 8, 128, 2, 128, 4, 32)
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.1)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32)
    raw = torch.empty(batch.packed_k.numel() + 8, dtype=torch.uint8, device=cuda_device)
    shifted = raw[8:].view(batch.packed_k.shape)
    shifted.copy_(batch.packed_k)
    moved = PackedBatch(shifted, batch.packed_v, batch.scales_k, batch.scales_v, batch.valid_tokens, 4, 32)
    auto = HipAttentionBackend("auto")
    out, lse = auto.run(query, moved, 0.1)
    assert auto.last_kernel == "general"
    check(out, lse, ref_out, ref_lse)
    for kernel in ("mfma", "staged"):
        with pytest.raises(ValueError, match="aligned"):
            HipAttentionBackend(kernel).run(query, moved, 0.1)


def test_int2_8_byte_aligned_buffers_use_mfma_kernel(cuda_device):
    # 8-byte aligned INT2 rows suit the register-staged kernel, not the 16-byte copies
    q, pk, pv, sk, sv, valid = make_batch(6, 32, 8, 128, 2, 128, 2, 32)
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 2, 32, 0.1)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 2, 32)
    raw = torch.empty(batch.packed_v.numel() + 8, dtype=torch.uint8, device=cuda_device)
    shifted = raw[8:].view(batch.packed_v.shape)
    shifted.copy_(batch.packed_v)
    moved = PackedBatch(batch.packed_k, shifted, batch.scales_k, batch.scales_v, batch.valid_tokens, 2, 32)
    auto = HipAttentionBackend("auto")
    out, lse = auto.run(query, moved, 0.1)
    assert auto.last_kernel == "mfma"
    check(out, lse, ref_out, ref_lse)


@pytest.mark.parametrize("bits", [2, 4])
def test_many_blocks_with_empty_and_partial_split_starts(cuda_device, bits):
    # 2048 blocks of 128 tokens: every split holds many blocks; zero and
    # partial valid counts at and right after split starts exercise the
    # staged kernel's early-copy speculation (first and second stage re-issued)
    rng = np.random.default_rng(41 + bits)
    nb = 2048
    q, pk, pv, sk, sv, _ = make_batch(5, 16, 4, 128, nb, 128, bits, 32)
    valid = rng.integers(1, 129, nb).astype(np.int32)
    valid[::4] = 0
    valid[1::8] = rng.integers(0, 3, nb // 8)
    valid[-5:] = 0
    for qdtype in (torch.float32, torch.float16):
        qq = torch.from_numpy(q).to(qdtype).float().numpy()
        ref_out, ref_lse = O.attention(qq, pk, pv, sk, sv, valid, bits, 32, 0.1, threads=16)
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype=qdtype)
        names = kernels_for(query, batch)
        assert "staged" in names
        for kernel in names:
            out, lse = HipAttentionBackend(kernel).run(query, batch, 0.1)
            check(out, lse, ref_out, ref_lse)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh"), [(8, 8), (32, 8), (64, 8), (48, 16)])
def test_staged_eight_kv_heads_per_workgroup(cuda_device, bits, qh, kvh):
    # kv_heads % 8 == 0 and at least 2048 (kv head, attended block) pairs: the
    # staged kernel gives each workgroup all 8 kv heads of a token row in
    # 64-token stages.  Empty blocks and valid counts inside the first stage
    # sit at split starts; the same blocks are then attended through a
    # scattered block table.
    rng = np.random.default_rng(1000 * bits + qh + kvh)
    nb = 2048 // kvh + 64
    q, pk, pv, sk, sv, _ = make_batch(7 + kvh, qh, kvh, 128, nb, 128, bits, 32)
    valid = rng.integers(1, 129, nb).astype(np.int32)
    valid[::4] = 0
    valid[1::8] = rng.integers(0, 3, nb // 8)
    valid[2::16] = rng.integers(60, 70, nb // 16)
    valid[-3:] = 0
    ids = [int(i) for i in rng.permutation(nb)[: 2048 // kvh + 40]]
    table = np.array(ids, np.int32)
    # (INT4 with 64 query heads and an fp32 / fp64 query takes 4 kv heads per
    # workgroup: the 8-kv-head form of those would not fit the registers)
    for qdtype in (torch.float32, torch.float64, torch.float16, torch.bfloat16):
        qq = torch.from_numpy(q).to(qdtype).float().numpy()
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype=qdtype)
        assert HipAttentionBackend("auto").kernel_for(query, batch) == "staged"
        for selection in (None, ids):
            ref_out, ref_lse = O.attention(
                qq, pk, pv, sk, sv, valid, bits, 32, 0.1, block_table=None if selection is None else table, threads=16
            )
            out, lse = HipAttentionBackend("staged").run(query, batch, 0.1, block_table=selection)
            check(out, lse, ref_out, ref_lse)


def test_merge_of_more_than_256_splits(cuda_device):
    # one kv head and 600 blocks: 600 splits, merged in batches of 256 with a
    # running rescale; the first 300 blocks (a whole batch and then some) hold
    # no valid token, and valid counts vary after that
    rng = np.random.default_rng(77)
    nb = 600
    q, pk, pv, sk, sv, _ = make_batch(9, 4, 1, 128, nb, 16, 4, 32)
    valid = rng.integers(0, 17, nb).astype(np.int32)
    valid[:300] = 0
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.2, threads=16)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32)
    for kernel in kernels_for(query, batch):
        out, lse = HipAttentionBackend(kernel).run(query, batch, 0.2)
        check(out, lse, ref_out, ref_lse)
    # every block empty: out 0, lse -inf
    empty = np.zeros(nb, np.int32)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, empty, 4, 32)
    out, lse = HipAttentionBackend("auto").run(query, batch, 0.2)
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))


@pytest.mark.parametrize("bits", [2, 4])
def test_staged_eight_kv_heads_stage_boundaries(cuda_device, bits):
    # 8 kv heads per workgroup with three groups (24 kv heads) and 256-token
    # blocks (four 64-token stages each): valid counts at and around stage
    # boundaries, and empty blocks at split starts
    rng = np.random.default_rng(500 + bits)
    nb, bt, kvh, qh = 100, 256, 24, 48
    q, pk, pv, sk, sv, _ = make_batch(31, qh, kvh, 128, nb, bt, bits, 32)
    edges = np.array([0, 1, 63, 64, 65, 127, 128, 129, 191, 192, 255, 256], np.int32)
    valid = edges[rng.integers(0, len(edges), nb)].astype(np.int32)
    valid[::5] = 0
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype=torch.float16)
    qq = torch.from_numpy(q).to(torch.float16).float().numpy()
    ref_out, ref_lse = O.attention(qq, pk, pv, sk, sv, valid, bits, 32, 0.1, threads=16)
    out, lse = HipAttentionBackend("staged").run(query, batch, 0.1)
    check(out, lse, ref_out, ref_lse)


def test_staged_eight_kv_heads_gqa8_reversed_table(cuda_device):
    # just past the 2048 (kv head, block) pairs that select 8 kv heads per
    # workgroup, GQA 8 (two query quads per wave), blocks attended in reverse
    # order through a table
    rng = np.random.default_rng(808)
    nb = 260
    q, pk, pv, sk, sv, _ = make_batch(44, 64, 8, 128, nb, 128, 4, 32)
    valid = rng.integers(1, 129, nb).astype(np.int32)
    ids = list(range(nb - 1, -1, -1))
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.1, block_table=np.array(ids, np.int32), threads=16)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32)
    out, lse = HipAttentionBackend("staged").run(query, batch, 0.1, block_table=ids)
    check(out, lse, ref_out, ref_lse)
    out, lse = HipAttentionBackend("staged").run(query, batch, 0.1)
    ref_out, ref_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.1, threads=16)
    check(out, lse, ref_out, ref_lse)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh", "nb"), [(48, 8, 12), (20, 4, 9), (64, 8, 80), (28, 4, 150)])
def test_mfma_query_quads_with_and_without_a_workgroup_each(cuda_device, bits, qh, kvh, nb):
    # More than 4 query heads per kv head (GQA 6, 5, 8, 7) on the matrix-core
    # kernel.  While 2 x splits x kv heads <= 1024 (one-block splits here),
    # each query quad gets a workgroup of its own, the second quad only partly
    # filled for GQA 5-7.  Beyond that (80 x 8 and 150 x 4 splits, with or
    # without a table) one workgroup carries both quads, the fp32 / fp64 INT4
    # form with registers spilled.  Every query dtype, empty blocks included.
    rng = np.random.default_rng(500 + bits + qh + nb)
    q, pk, pv, sk, sv, _ = make_batch(71 + nb, qh, kvh, 128, nb, 128, bits, 32)
    valid = rng.integers(0, 129, nb).astype(np.int32)
    ids = [int(i) for i in rng.permutation(nb)[: max(1, nb - 3)]]
    for qdtype in (torch.float16, torch.bfloat16, torch.float32, torch.float64):
        qq = torch.from_numpy(q).to(qdtype).float().numpy()
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype=qdtype)
        for selection in (None, ids):
            table = None if selection is None else np.array(selection, np.int32)
            ref_out, ref_lse = O.attention(qq, pk, pv, sk, sv, valid, bits, 32, 0.1, block_table=table, threads=16)
            out, lse = HipAttentionBackend("mfma").run(query, batch, 0.1, block_table=selection)
            check(out, lse, ref_out, ref_lse)


@pytest.mark.parametrize("qdtype", [torch.float16, torch.bfloat16, torch.float32, torch.float64])
@pytest.mark.parametrize("bits", [2, 4])
def test_output_in_query_dtype_is_the_rounded_fp32_output(cuda_device, qdtype, bits):
    """out_dtype=query.dtype stores what out.to(query.dtype) gives, bit for bit
    (torch rounds fp32 to fp16 / bf16 to nearest even), for every kernel, a
    merge of more than 64 splits (600 blocks of one kv head) and empty blocks."""
    cases = [make_batch(61 + bits, 32, 8, 128, 6, 128, bits, 32), make_batch(62, 4, 1, 128, 600, 16, bits, 32)]
    cases[1] = cases[1][:5] + (np.where(np.arange(600) % 7 == 0, 0, cases[1][5]).astype(np.int32),)
    for q, pk, pv, sk, sv, valid in cases:
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, qdtype)
        for kernel in kernels_for(query, batch):
            backend = HipAttentionBackend(kernel)
            out32, lse32 = backend.run(query, batch, 0.1)
            outq, lseq = backend.run(query, batch, 0.1, out_dtype=qdtype)
            assert out32.dtype == torch.float32 and outq.dtype == qdtype and lseq.dtype == torch.float32
            assert torch.equal(outq, out32.to(qdtype)), kernel
            assert torch.equal(lseq, lse32), kernel
    # no valid token: 0 in every dtype, lse -inf
    q, pk, pv, sk, sv, _ = cases[0]
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, np.zeros(6, np.int32), bits, 32, qdtype)
    outq, lseq = HipAttentionBackend("auto").run(query, batch, 0.1, out_dtype=qdtype)
    assert torch.all(outq == 0) and torch.all(torch.isneginf(lseq))
    other = torch.bfloat16 if qdtype == torch.float16 else torch.float16
    with pytest.raises(ValueError, match="out_dtype"):
        HipAttentionBackend("auto").run(query, batch, 0.1, out_dtype=other)


def test_two_phase_entry_points_write_the_query_dtype(cuda_device):
    """kvssd_hip_decode_partials + kvssd_hip_decode_merge with out_query_dtype=1
    give the fused call's typed output."""
    q, pk, pv, sk, sv, valid = make_batch(63, 32, 8, 128, 40, 128, 4, 32)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32, torch.bfloat16)
    backend = HipAttentionBackend("auto")
    fused, fused_lse = backend.run(query, batch, 0.1, out_dtype=torch.bfloat16)
    lib = _native.load()
    desc = backend.describe(query, batch, 0.1)
    desc.out_query_dtype = 1
    need = ctypes.c_size_t(0)
    _native.check(lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(need)), "workspace")
    work = torch.empty(need.value, dtype=torch.uint8, device=cuda_device)
    out = torch.empty(32, 128, dtype=torch.bfloat16, device=cuda_device)
    lse = torch.empty(32, dtype=torch.float32, device=cuda_device)
    stream = _native.stream_handle(torch.cuda.current_stream(cuda_device))
    args = [t.data_ptr() for t in (query, batch.packed_k, batch.packed_v, batch.scales_k, batch.scales_v,
                                   batch.valid_tokens)]
    _native.check(lib.kvssd_hip_decode_partials(ctypes.byref(desc), *args, None, work.data_ptr(), need.value, stream),
                  "decode_partials")
    _native.check(lib.kvssd_hip_decode_merge(ctypes.byref(desc), work.data_ptr(), need.value, out.data_ptr(),
                                             lse.data_ptr(), stream), "decode_merge")
    torch.cuda.synchronize()
    assert torch.equal(out, fused) and torch.equal(lse, fused_lse)


def test_prepared_decode_fast_call_and_ctypes_agree(cuda_device):
    """A prepared decode launches through the CPython fast-call module when it
    is built and through the ctypes function otherwise: both call the same
    entry point with the same arguments, so their outputs are bit-equal (and
    match the oracle), for the staged and the matrix-core kernels, with and
    without a block table, and more calls than one block of output rows."""
    assert _native.fused_decode_fast() is not None, "the fast-call module is built with the library"
    rng = np.random.default_rng(17)
    # (INT2 with 4 query heads per kv head: the scores on the fp6 x fp4 core)
    for bits, nb, qh, kvh in ((4, 40, 32, 8), (2, 24, 16, 4)):
        q, pk, pv, sk, sv, valid = make_batch(18 + bits, qh, kvh, 128, nb, 128, bits, 32)
        q = torch.from_numpy(q).to(torch.float16).float().numpy()  # the values the kernel sees
        query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, bits, 32, torch.float16)
        for table in (None, [int(i) for i in rng.permutation(nb)[: nb // 2]]):
            ref_out, ref_lse = O.attention(
                q, pk, pv, sk, sv, valid, bits, 32, 0.1, block_table=None if table is None else np.array(table, np.int32)
            )
            for kernel in ("staged", "mfma"):
                fast = HipAttentionBackend(kernel).prepare(query, batch, 0.1, block_table=table)
                slow = HipAttentionBackend(kernel).prepare(query, batch, 0.1, block_table=table)
                assert fast._fast is not None
                slow._fast = None  # the ctypes route
                outs = [fast(query) for _ in range(70)] + [slow(query) for _ in range(70)]
                torch.cuda.synchronize()
                for out, lse in outs[1:]:
                    assert torch.equal(out, outs[0][0]) and torch.equal(lse, outs[0][1])
                check(outs[0][0], outs[0][1], ref_out, ref_lse)


def test_prepared_decode_matches_run(cuda_device):
    """HipAttentionBackend.prepare: repeated calls (one workspace per stream),
    a call on a second stream, the typed output and a block table give run's
    results bit for bit; a query of another shape or dtype is refused."""
    rng = np.random.default_rng(91)
    q, pk, pv, sk, sv, valid = make_batch(92, 32, 8, 128, 40, 128, 4, 32)
    query, batch = to_device(cuda_device, q, pk, pv, sk, sv, valid, 4, 32, torch.float16)
    backend = HipAttentionBackend("auto")
    for table in (None, [int(i) for i in rng.permutation(40)[:17]]):
        ref_out, ref_lse = backend.run(query, batch, 0.1, block_table=table)
        prepared = backend.prepare(query, batch, 0.1, block_table=table)
        for _ in range(3):
            out, lse = prepared(query)
            assert torch.equal(out, ref_out) and torch.equal(lse, ref_lse)
        side = torch.cuda.Stream(cuda_device)
        side.wait_stream(torch.cuda.current_stream(cuda_device))
        with torch.cuda.stream(side):
            out2, lse2 = prepared(query)
        torch.cuda.current_stream(cuda_device).wait_stream(side)
        assert torch.equal(out2, ref_out) and torch.equal(lse2, ref_lse)
        assert len(prepared._slots) == 2
        # the signature check without launching
        assert prepared.try_call(query.float()) is None and prepared.try_call(query[:16]) is None
        typed = backend.prepare(query, batch, 0.1, block_table=table, out_dtype=torch.float16)
        out16, _ = typed(query)
        assert out16.dtype == torch.float16 and torch.equal(out16, ref_out.to(torch.float16))
    # a new query of the same shape is decoded afresh
    other = torch.randn(32, 128, generator=torch.Generator().manual_seed(3)).to(torch.float16).to(cuda_device)
    assert torch.equal(prepared(other)[0], backend.run(other, batch, 0.1, block_table=table)[0])
    with pytest.raises(ValueError, match="does not match"):
        prepared(query.float())
    with pytest.raises(ValueError, match="does not match"):
        prepared(query[:16])
