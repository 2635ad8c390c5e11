"""Value range of the matrix-core kernels' fp16 softmax weights.

The reference computes softmax(s) V in fp32 (src/kvssd/backends/reference.py:
29-32, 46-49).  The matrix-core kernels form W = p * scale_v in fp16 for the PV
product, so without care W overflows for large V scales (the staged INT4
kernel's fine slots carry 16 p scale_v: a scale above 4,095 gave inf, then
NaN outputs) and falls into fp16's subnormals for tiny ones (precision lost).
Every stage therefore normalises W by a power of two set by its largest V
scale (csrc/common.hpp, wave_scale_exp).  These cases pin the whole range at
131,072 tokens (1,024 blocks of 128, 8 kv heads, 32 query heads), INT4 and
INT2, on every kernel:

* V scaled by 1e-5, 1e-3 and 1 (fp16 inputs, so 1e-5 puts V itself among
  fp16's subnormals), under spread attention (random keys: ~uniform weights)
  and under peaked attention (64 needles carrying ~99 % of the softmax mass);
* V groups whose max |v| is 30,000-60,000 (2 % of all groups, plus needles of
  value 50,000 under peaked attention), where the reference stays finite.

Checks: finite outputs; out at norm-relative error 1e-2; lse at max-abs 2e-3;
the contract tolerance (rel 1e-2, max-abs 2e-3 times the output's magnitude
where that exceeds 1: fp16 outputs of magnitude 1e4 are spaced by 8, so an
absolute 2e-3 cannot apply there).  A negative control shows the check fails
against the oracle with one needle dropped.

Inputs are quantised by the library's GPU quantiser (bit-identical to the
oracle's, tests/test_gpu_records.py): the CPU quantiser spends ~20 s on a
tensor of fp16 subnormals.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import needles as N
from kvssd.backends import PackedBatch
from oracle import oracle as O
from kvssd import records_hip
from kvssd.backends.hip import HipAttentionBackend

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)
TOKENS, NB, BT, KVH, QH, D = 131072, 1024, 128, 8, 32, 128
KERNELS = ("general", "mfma", "staged")
NEEDLES = 64


def make_base() -> dict:
    """fp16-representable K, V [T, KVH, D] (float32), an fp16 query, the
    needles' (block, row) positions, keys and unit values, and the large-V
    groups."""
    rng = np.random.default_rng(31337)
    k = (0.5 * rng.standard_normal((TOKENS, KVH, D), dtype=np.float32)).astype(np.float16).astype(np.float32)
    v = rng.standard_normal((TOKENS, KVH, D), dtype=np.float32).astype(np.float16).astype(np.float32)
    q = rng.standard_normal((QH, D)).astype(np.float16)
    # one needle per 16 blocks (every split of every kernel's plan holds some)
    blocks = np.arange(NEEDLES) * (NB // NEEDLES) + rng.integers(0, NB // NEEDLES, NEEDLES)
    rows = rng.integers(0, BT, NEEDLES)
    keys = N.needle_keys(q.astype(np.float32), KVH, SCALE, target=12.0)
    unit = N.needle_values(NEEDLES, KVH, D, 1.0, rng)
    large = rng.random((TOKENS, KVH, D // 32)) < 0.02
    large_max = rng.uniform(30000.0, 60000.0, large.shape).astype(np.float32)
    return dict(k=k, v=v, q=q, blocks=blocks, rows=rows, keys=keys, unit=unit, large=large, large_max=large_max)


def quantize_blocks(x: np.ndarray, bits: int, dev) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """(packed [NB, BT, KVH, PD], fp16 scales [NB, BT, KVH, 4], valid) of [T, KVH, D] values."""
    q = records_hip.quantize(torch.from_numpy(x).to(dev), bits, 32)
    packed = q.packed.cpu().numpy().reshape(NB, BT, KVH, D * bits // 8)
    scales = q.scales.cpu().numpy().reshape(NB, BT, KVH, D // 32)
    return packed, scales, np.full(NB, BT, np.int32)


def make_keys(base: dict, bits: int, dev) -> dict:
    """Quantised K for one bit width: random keys (spread) and with the needle keys (peaked)."""
    k4 = base["k"].reshape(NB, BT, KVH, D)
    spread = quantize_blocks(base["k"], bits, dev)
    kn = k4.copy()
    kn[base["blocks"], base["rows"]] = base["keys"][None].astype(np.float16).astype(np.float32)
    peaked = quantize_blocks(kn.reshape(TOKENS, KVH, D), bits, dev)
    return {"spread": spread, "peaked": peaked}


@pytest.fixture(scope="module")
def base():
    return make_base()


@pytest.fixture(scope="module", params=[4, 2])
def keys_q(request, base, cuda_device):
    return request.param, make_keys(base, request.param, cuda_device)


def values(base, pattern: str, vscale: float) -> np.ndarray:
    """V [T, KVH, D] for a case, fp16-representable."""
    if vscale == "large":
        g = base["v"].reshape(TOKENS, KVH, D // 32, 32) * 0.5
        gmax = np.maximum(np.abs(g).max(axis=-1, keepdims=True), 1e-3)
        g = np.where(base["large"][..., None], g / gmax * base["large_max"][..., None], g)
        v = g.reshape(TOKENS, KVH, D)
        amp = 50000.0
    else:
        v = base["v"] * np.float32(vscale)
        amp = 8.0 * vscale
    v = v.astype(np.float16).astype(np.float32)
    if pattern == "peaked":
        v4 = v.reshape(NB, BT, KVH, D)
        v4[base["blocks"], base["rows"]] = (base["unit"] * np.float32(amp)).astype(np.float16).astype(np.float32)
    return v


def run_kernels(dev, q16, arrays, valid, bits):
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in arrays), torch.from_numpy(valid).to(dev), bits, 32)
    out = {}
    for kernel in KERNELS:
        o, l = HipAttentionBackend(kernel).run(torch.from_numpy(q16).to(dev), batch, SCALE)
        out[kernel] = (o.cpu().numpy(), l.cpu().numpy())
    return out


def assert_range_match(out, lse, ref_out, ref_lse, what):
    assert np.isfinite(out).all() and np.isfinite(lse).all(), f"{what}: non-finite output"
    mag = max(1.0, float(np.abs(ref_out).max()))
    excess = float(np.max(np.abs(out - ref_out) - N.RTOL * np.abs(ref_out)))
    lse_abs = float(np.max(np.abs(lse - ref_lse)))
    norm_rel = float(np.linalg.norm(out - ref_out) / max(np.linalg.norm(ref_out), 1e-30))
    msg = f"{what}: out excess {excess:.3e} (bound {N.ATOL * mag:.3e}), |dlse| {lse_abs:.3e}, norm-rel {norm_rel:.3e}"
    assert excess <= N.ATOL * mag, msg
    assert lse_abs <= N.LSE_ATOL, msg
    assert norm_rel <= N.NORM_RTOL, msg
    return norm_rel


@pytest.mark.parametrize("pattern", ["spread", "peaked"])
@pytest.mark.parametrize("vscale", [1e-5, 1e-3, 1.0, "large"])
def test_value_range_128k_tokens(cuda_device, base, keys_q, vscale, pattern):
    bits, kq = keys_q
    pk, sk, valid = kq[pattern]
    pv, sv, _ = quantize_blocks(values(base, pattern, vscale), bits, cuda_device)
    arrays = [pk, pv, sk, sv]
    q16 = base["q"]
    ref_out, ref_lse = N.oracle(q16.astype(np.float32), arrays, valid, bits)
    assert np.isfinite(ref_out).all(), "the oracle itself is finite on these inputs"
    what = f"INT{bits} V x{vscale} {pattern}"
    results = run_kernels(cuda_device, q16, arrays, valid, bits)
    for kernel, (out, lse) in results.items():
        assert_range_match(out, lse, ref_out, ref_lse, f"{what} {kernel}")
    if pattern == "peaked":
        # dropping one needle (its row moved past the block's valid count)
        # must fail the same check: each needle carries ~1/64 of the mass
        b, r = int(base["blocks"][NEEDLES // 2]), int(base["rows"][NEEDLES // 2])
        v2 = valid.copy()
        v2[b] -= 1
        c_out, c_lse = N.oracle(q16.astype(np.float32), N.move_rows_to_end(arrays, b, [r]), v2, bits)
        for kernel, (out, lse) in results.items():
            norm_rel = float(np.linalg.norm(out - c_out) / np.linalg.norm(c_out))
            assert norm_rel > 2 * N.NORM_RTOL, f"{what} {kernel}: the check would pass with one needle dropped"


def large_score_case(bits: int, nb: int, mult: float, outliers: bool):
    """Peaked attention with large scores: one needle token per kv head whose
    key points along the sum of the head's query group; the query scaled by
    ``mult`` (largest lse ~ 30-40 mult with outliers, ~ 7-8 mult without), with
    one dim per 32-dim group 20 times the others when ``outliers``."""
    rng = np.random.default_rng(9)
    kvh, qh, d, bt = 8, 32, 128, 128
    k = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    v = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    q0 = rng.standard_normal((qh, d)).astype(np.float32)
    qs = q0.reshape(kvh, qh // kvh, d).sum(1)
    needle = (nb * bt) // 3
    k[needle] = qs / np.linalg.norm(qs, axis=1, keepdims=True) * math.sqrt(d)
    pk, sk, _ = O.quantize_blocks(k, bits, 32, bt)
    pv, sv, _ = O.quantize_blocks(v, bits, 32, bt)
    q = q0 * np.float32(mult)
    if outliers:
        q[:, 5::32] *= 20
    q16 = q.astype(np.float16)
    return q16, [pk, pv, sk, sv], np.full(nb, bt, np.int32)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("nb", [64, 256])
def test_large_scores_and_query_outliers(cuda_device, bits, nb):
    # The reference scores in fp32 (src/kvssd/backends/reference.py:42-45): a
    # plain fp32 dot product and logsumexp stay within 1e-4 of float64 here
    # even at lse ~ 1,300.  A kernel whose query operand kept only a fixed
    # number of bits relative to a 32-dim block's largest value errs in
    # proportion to the scores: three block-scaled fp6 parts missed lse by
    # 2.5e-3 at lse ~ 29 with the outlier dims (64 blocks) and by 3.8e-3 at
    # lse ~ 41 (256 blocks).  The cases stop at lse ~ 250: beyond that the
    # staged INT2 scores, which remove the codes' offset through the fp32
    # accumulator, round by more than 2e-3 in absolute terms (3.8e-3 at lse
    # ~ 1,300, 2.9e-6 relative).  64 blocks take the staged kernel's 4-kv-head
    # workgroups, 256 blocks its 8-kv-head ones.
    scale = 1 / math.sqrt(128)
    for mult, outliers in ((1.0, True), (4.0, True), (16.0, False), (32.0, False)):
        q16, arrays, valid = large_score_case(bits, nb, mult, outliers)
        qf = q16.astype(np.float32)
        ref_out, ref_lse = O.attention(qf, *arrays, valid, bits, 32, scale)
        batch = PackedBatch(*(torch.from_numpy(a).to(cuda_device) for a in arrays),
                            torch.from_numpy(valid).to(cuda_device), bits, 32)
        for kernel in KERNELS:
            backend = HipAttentionBackend(kernel)
            out, lse = backend.run(torch.from_numpy(q16).to(cuda_device), batch, scale)
            what = f"INT{bits} {nb} blocks x{mult} outliers={outliers} {kernel} (lse up to {ref_lse.max():.0f})"
            assert_range_match(out.cpu().numpy(), lse.cpu().numpy(), ref_out, ref_lse, what)


@pytest.mark.parametrize("bits", [2, 4])
def test_unusual_softmax_scales(cuda_device, bits):
    # sm_scale is any float the caller passes (src/kvssd/backends/reference.py:
    # 42-45 multiplies the scores by it): zero (uniform weights, lse = ln of the
    # token count, out = the mean of the values), tiny, larger than 1/sqrt(D)
    # and negative, on every kernel, 64 blocks (the staged kernel's 4-kv-head
    # workgroups) and 256 (its 8-kv-head ones)
    rng = np.random.default_rng(3)
    for nb in (64, 256):
        k = rng.standard_normal((nb * 128, 8, 128)).astype(np.float32)
        v = rng.standard_normal((nb * 128, 8, 128)).astype(np.float32)
        pk, sk, _ = O.quantize_blocks(k, bits, 32, 128)
        pv, sv, _ = O.quantize_blocks(v, bits, 32, 128)
        valid = np.full(nb, 128, np.int32)
        valid[nb // 2] = 77  # one partial block
        q16 = rng.standard_normal((32, 128)).astype(np.float16)
        batch = PackedBatch(*(torch.from_numpy(a).to(cuda_device) for a in (pk, pv, sk, sv, valid)), bits, 32)
        for scale in (0.0, 1e-4, 0.5, 2.0, -0.1):
            ref_out, ref_lse = O.attention(q16.astype(np.float32), pk, pv, sk, sv, valid, bits, 32, scale)
            if scale == 0.0:
                # the closed form the oracle must meet first
                n = int(valid.sum())
                assert np.allclose(ref_lse, math.log(n), atol=1e-6)
                vals = O.dequantize_np(O.unpack_np(pv, bits), sv, bits, 32).reshape(nb, 128, 8, 128)
                mean = np.concatenate([vals[b, : valid[b]] for b in range(nb)]).mean(0)  # [8, 128]
                assert np.allclose(ref_out, np.repeat(mean, 4, axis=0), atol=1e-5)
            for kernel in KERNELS:
                out, lse = HipAttentionBackend(kernel).run(torch.from_numpy(q16).to(cuda_device), batch, scale)
                what = f"INT{bits} {nb} blocks sm_scale {scale} {kernel} (lse up to {ref_lse.max():.0f})"
                assert_range_match(out.cpu().numpy(), lse.cpu().numpy(), ref_out, ref_lse, what)
