"""GPU record codec against the CPU oracle, through the C ABI.

Bars: bit-exact bytes for packed codes, fp16 scales, whole records and
CRC-32 values (integer/byte work); the oracle's quantiser and record encoder
are pinned by tests/test_golden.py and tests/test_oracle.py (closed forms,
zlib.crc32 and the check value crc32(b"123456789") == 0xCBF43926).
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

TORCH_DTYPES = [torch.float16, torch.bfloat16, torch.float32, torch.float64]


def oracle_quantize(x: torch.Tensor, bits: int, g: int) -> tuple[np.ndarray, np.ndarray]:
    # the 1e30 edge row overflows the fp16 scale to inf on purpose (as torch's cast does)
    with np.errstate(over="ignore"):
        codes, scales = O.quantize_np(x.float().cpu().numpy(), bits, g)
    return O.pack_np(codes, bits), scales


def edge_rows(d: int, g: int, dtype: torch.dtype) -> torch.Tensor:
    """Rows that exercise the quantiser's corners: zeros, -0, exact .5 ties,
    tiny groups (scale clamp), the fp16 maximum, single spikes."""
    rows = [
        torch.zeros(d),
        -torch.zeros(d),
        torch.full((d,), 1e-12),
        torch.linspace(-7.0, 7.0, d),            # ties land on x/scale = k + 0.5 for some k
        # max 7 makes the INT4 scale exactly 1: every other value is a .5 tie
        torch.cat([torch.tensor([7.0]), torch.arange(d - 1, dtype=torch.float32) % 8 - 3.5]),
        torch.full((d,), 65504.0 if dtype == torch.float16 else 1e30),
    ]
    spike = torch.zeros(d)
    spike[::g] = 3.0
    rows.append(spike)
    return torch.stack(rows).to(dtype)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("g", [16, 32])
@pytest.mark.parametrize("dtype", TORCH_DTYPES)
def test_quantize_bit_exact(cuda_device, bits, g, dtype):
    gen = torch.Generator().manual_seed(5 + bits + g)
    x = (torch.randn(513, 128, generator=gen) * 3).to(dtype)
    x = torch.cat([x, edge_rows(128, g, dtype)])
    q = R.quantize(x.to(cuda_device), bits, g)
    packed, scales = oracle_quantize(x, bits, g)
    assert np.array_equal(q.packed.cpu().numpy(), packed)
    assert np.array_equal(q.scales.cpu().numpy().view(np.uint16), scales.view(np.uint16))
    assert q.original_shape == tuple(x.shape)


def test_quantize_matches_product_quantizer(cuda_device):
    # the product's CPU quantize_tensor (itself pinned to the reference's
    # closed form) and the GPU twin agree on a 3-D KV tensor
    from kvssd.quant import quantize_tensor

    gen = torch.Generator().manual_seed(3)
    x = torch.randn(64, 8, 128, generator=gen, dtype=torch.float16)
    cpu = quantize_tensor(x, 4, 32)
    gpu = R.quantize(x.to(cuda_device), 4, 32)
    assert torch.equal(cpu.packed, gpu.packed.cpu())
    assert torch.equal(cpu.scales.view(torch.int16), gpu.scales.cpu().view(torch.int16))


def oracle_records(keys: np.ndarray, values: np.ndarray, spec: CacheSpec, layer: int, first_block: int) -> list[bytes]:
    """Records as KVCacheStore.create writes them (zero-padded last block)."""
    t = keys.shape[0]
    bt = spec.block_tokens
    pk, sk, valid = O.quantize_blocks(keys, spec.bits, spec.group_size, bt)
    pv, sv, _ = O.quantize_blocks(values, spec.bits, spec.group_size, bt)
    out = []
    for b in range(pk.shape[0]):
        out.append(
            O.encode_record(
                layer, first_block + b, int(valid[b]), spec.bits, bt, spec.kv_heads, spec.head_dim, spec.group_size,
                sk[b], sv[b], pk[b], pv[b],
            )
        )
    assert t == sum(int(v) for v in valid)
    return out


SPECS = [
    CacheSpec(layers=1, kv_heads=8, head_dim=128, block_tokens=128, bits=4, group_size=32),
    CacheSpec(layers=1, kv_heads=8, head_dim=128, block_tokens=128, bits=2, group_size=32),
    CacheSpec(layers=1, kv_heads=2, head_dim=64, block_tokens=32, bits=4, group_size=16),
    # payload of 6 * BT * KVH = 18 bytes: not a multiple of 4 (byte paths)
    CacheSpec(layers=1, kv_heads=1, head_dim=4, block_tokens=3, bits=2, group_size=4),
    # 55,296-byte payload: 4 rows of 16-byte chunks behind 10,240 virtual zero bytes
    CacheSpec(layers=1, kv_heads=8, head_dim=128, block_tokens=48, bits=4, group_size=32),
    # 294,912-byte payload: beyond the chunked form's 256 KiB, general form
    CacheSpec(layers=1, kv_heads=8, head_dim=128, block_tokens=256, bits=4, group_size=32),
]


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: f"b{s.bits}-kvh{s.kv_heads}-d{s.head_dim}-bt{s.block_tokens}")
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_encode_records_bit_exact(cuda_device, spec, dtype):
    gen = torch.Generator().manual_seed(11)
    tokens = 3 * spec.block_tokens - 1  # partial last block
    k = torch.randn(tokens, spec.kv_heads, spec.head_dim, generator=gen).to(dtype)
    v = torch.randn(tokens, spec.kv_heads, spec.head_dim, generator=gen).to(dtype)
    recs, crcs = R.encode_records(k.to(cuda_device), v.to(cuda_device), spec, layer=5, first_block=7)
    want = oracle_records(k.float().numpy(), v.float().numpy(), spec, 5, 7)
    got = recs.cpu().numpy()
    assert got.shape == (len(want), spec.record_bytes)
    for i, w in enumerate(want):
        assert got[i].tobytes() == w, f"record {i} differs"
        assert int(crcs[i]) == int.from_bytes(w[48:52], "little")
        assert int(crcs[i]) == zlib.crc32(w[52 : 52 + int.from_bytes(w[44:48], "little")])


def device_records(recs: list[bytes], device) -> torch.Tensor:
    return torch.from_numpy(np.frombuffer(b"".join(recs), dtype=np.uint8).copy()).to(device)


@pytest.mark.parametrize("spec", SPECS, ids=lambda s: f"b{s.bits}-kvh{s.kv_heads}-d{s.head_dim}-bt{s.block_tokens}")
def test_gather_records_bit_exact(cuda_device, spec):
    rng = np.random.default_rng(2)
    tokens = 4 * spec.block_tokens - 2
    k = rng.standard_normal((tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    v = rng.standard_normal((tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    recs = oracle_records(k, v, spec, 0, 0)
    raw = device_records(recs, cuda_device)
    pk, pv, sk, sv, valid, status = R.gather_records(raw, spec, len(recs))
    opk, osk, ovalid = O.quantize_blocks(k, spec.bits, spec.group_size, spec.block_tokens)
    opv, osv, _ = O.quantize_blocks(v, spec.bits, spec.group_size, spec.block_tokens)
    assert status.cpu().tolist() == [R.OK] * len(recs)
    assert np.array_equal(valid.cpu().numpy(), ovalid)
    assert np.array_equal(pk.cpu().numpy(), opk)
    assert np.array_equal(pv.cpu().numpy(), opv)
    assert np.array_equal(sk.cpu().numpy().view(np.uint16), osk.view(np.uint16))
    assert np.array_equal(sv.cpu().numpy().view(np.uint16), osv.view(np.uint16))


def test_gather_records_detects_corruption(cuda_device):
    spec = SPECS[0]
    rng = np.random.default_rng(4)
    k = rng.standard_normal((6 * spec.block_tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    recs = [bytearray(r) for r in oracle_records(k, k, spec, 2, 10)]
    recs[1][52 + 1000] ^= 0x01                     # payload bit flip -> CRC
    recs[2][0:8] = b"KVSSD002"                     # magic
    recs[3][8:12] = (2).to_bytes(4, "little")      # version
    recs[4][24:28] = (2).to_bytes(4, "little")     # bits: layout differs
    recs[5][44:48] = (1234).to_bytes(4, "little")  # payload length
    raw = device_records([bytes(r) for r in recs], cuda_device)
    *_, status = R.gather_records(raw, spec, len(recs))
    assert status.cpu().tolist() == [R.OK, R.BAD_CRC, R.BAD_HEADER, R.BAD_HEADER, R.BAD_LAYOUT, R.BAD_CRC]
    with pytest.raises(IOError, match="CRC mismatch for layer=2, block=11"):
        R.raise_for_status(status, 2, list(range(10, 16)))
    # without verification a flipped payload byte passes (and is copied as is)
    *_, status = R.gather_records(raw[: 2 * spec.record_bytes], spec, 2, verify_crc=False)
    assert status.cpu().tolist() == [R.OK, R.OK]


def test_gather_then_decode_matches_oracle(cuda_device):
    # records -> GPU gather -> fused decode equals the oracle on the same blocks
    from kvssd.backends import PackedBatch
    from kvssd.backends.hip import HipAttentionBackend

    spec = SPECS[0]
    rng = np.random.default_rng(8)
    tokens = 5 * spec.block_tokens - 17
    k = rng.standard_normal((tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    v = rng.standard_normal((tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    q = rng.standard_normal((32, spec.head_dim)).astype(np.float32)
    raw = device_records(oracle_records(k, v, spec, 0, 0), cuda_device)
    pk, pv, sk, sv, valid, status = R.gather_records(raw, spec, -(-tokens // spec.block_tokens))
    assert int(status.max()) == R.OK
    out, lse = HipAttentionBackend().run(torch.from_numpy(q).to(cuda_device), PackedBatch(pk, pv, sk, sv, valid, 4, 32), 0.1)
    opk, osk, ovalid = O.quantize_blocks(k, 4, 32, spec.block_tokens)
    opv, osv, _ = O.quantize_blocks(v, 4, 32, spec.block_tokens)
    ref_out, ref_lse = O.attention(q, opk, opv, osk, osv, ovalid, 4, 32, 0.1)
    np.testing.assert_allclose(out.cpu().numpy(), ref_out, atol=2e-3, rtol=1e-2)
    np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-3, rtol=1e-2)


def test_gather_records_unaligned_outputs(cuda_device):
    # outputs that are not 16-byte aligned take the general form; same bytes
    spec = SPECS[0]
    rng = np.random.default_rng(6)
    k = rng.standard_normal((3 * spec.block_tokens, spec.kv_heads, spec.head_dim)).astype(np.float32)
    recs = oracle_records(k, k[::-1].copy(), spec, 0, 0)
    raw = device_records(recs, cuda_device)
    want = R.gather_records(raw, spec, 3)
    n, bt, kvh = 3, spec.block_tokens, spec.kv_heads
    pbytes = n * bt * kvh * spec.packed_dim
    sbytes = n * bt * kvh * (spec.head_dim // spec.group_size) * 2
    buf = torch.zeros(2 * pbytes + 2 * sbytes + 64, dtype=torch.uint8, device=cuda_device)
    pk = buf[4 : 4 + pbytes].view(n, bt, kvh, spec.packed_dim)
    pv = buf[8 + pbytes : 8 + 2 * pbytes].view(n, bt, kvh, spec.packed_dim)
    base = 16 + 2 * pbytes
    sk = buf[base : base + sbytes].view(torch.float16).view(n, bt, kvh, -1)
    sv = buf[base + sbytes + 8 : base + 2 * sbytes + 8].view(torch.float16).view(n, bt, kvh, -1)
    valid = torch.empty(n, dtype=torch.int32, device=cuda_device)
    status = torch.empty(n, dtype=torch.int32, device=cuda_device)
    got = R.gather_records(raw, spec, n, out=(pk, pv, sk, sv, valid, status))
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.uint8) if a.dtype == torch.float16 else a, b.view(torch.uint8) if b.dtype == torch.float16 else b)


@pytest.mark.parametrize("bits", [2, 4])
def test_quantize_unaligned_source_matches(cuda_device, bits):
    # a source that is not 16-byte aligned takes the element-wise form; the
    # register form (aligned, group 32) gives the same bytes
    gen = torch.Generator().manual_seed(21)
    x = torch.randn(301, 128, generator=gen).half()
    buf = torch.empty(301 * 128 + 1, dtype=torch.float16, device=cuda_device)
    shifted = buf[1:].view(301, 128)
    shifted.copy_(x.to(cuda_device))
    a = R.quantize(shifted, bits, 32)
    b = R.quantize(x.to(cuda_device), bits, 32)
    packed, scales = oracle_quantize(x, bits, 32)
    assert torch.equal(a.packed, b.packed) and np.array_equal(a.packed.cpu().numpy(), packed)
    assert np.array_equal(a.scales.cpu().numpy().view(np.uint16), scales.view(np.uint16))
