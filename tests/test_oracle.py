"""Pins for the CPU oracle (oracle/): every oracle function is checked against
something that does not restate its own formula: a library routine, a closed
form, an exhaustive sweep, brute force on tiny inputs, or an invariant chosen so
that a plausible mistake (dropped term, wrong sign or index, transposed operand)
fails it.

Oracle function              pinned by
---------------------------  ------------------------------------------------
orc_f16_to_f32               numpy float16 -> float32 over all 65536 halves
orc_f32_to_f16               numpy float32 -> float16 (round to nearest even)
                             over a dense sweep incl. subnormals, ties, overflow
orc_crc32                    zlib.crc32 and crc32(b"123456789") == 0xCBF43926
quantize (C and numpy)       closed-form known answers (half-even ties, all-zero
                             group, INT2 group), invariants, the reference's MAE
                             bounds (tests/test_quant.py:7)
pack / unpack                known answers + exhaustive byte sweep
attention                    torch float64 scaled_dot_product_attention on the
                             dequantised tensors; single-token and equal-key
                             closed forms; pure-Python brute force
merge                        split-anywhere invariant against one full call
selectors                    closed-form known answers
record format                struct layout, CacheSpec sizes (151552 / 86016)
vLLM block record            hand-assembled known answer (header fields, scale
                             and code bytes, zlib CRC, padding); decode of the
                             known answer gives the closed-form values; decode
                             inverts encode to within half a quantisation step
"""

from __future__ import annotations

import math
import struct
import zlib

import numpy as np
import pytest
import torch

from oracle import oracle as O


# ------------------------------------------------------------------ fp16 ---


def test_f16_to_f32_all_halves():
    lib = O.lib()
    halves = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = halves.view(np.float16).astype(np.float32)
    got = np.array([lib.orc_f16_to_f32(int(h)) for h in halves], dtype=np.float32)
    same = (got == ref) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_matches_numpy_round_to_nearest_even():
    lib = O.lib()
    rng = np.random.default_rng(0)
    mags = rng.standard_normal(40000).astype(np.float32) * (
        np.float32(2.0) ** rng.integers(-30, 18, 40000).astype(np.float32)
    )
    # exact ties between adjacent halves, subnormal ties, overflow boundary
    halves = np.arange(0, 0x7C00, 7, dtype=np.uint16).view(np.float16).astype(np.float64)
    ties = ((halves[:-1] + halves[1:]) / 2).astype(np.float32)
    specials = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e-8, 2.0**-25, 2.0**-24, 6e-8, -3e-5], np.float32)
    xs = np.concatenate([mags, ties, specials])
    with np.errstate(over="ignore"):
        ref = xs.astype(np.float16).view(np.uint16)
    got = np.array([lib.orc_f32_to_f16(float(v)) for v in xs], dtype=np.uint16)
    assert np.array_equal(got, ref)


def test_crc32_known_answer_and_zlib():
    assert O.crc32(b"123456789") == 0xCBF43926
    data = np.random.default_rng(1).integers(0, 256, 100_003, dtype=np.uint8).tobytes()
    assert O.crc32(data) == zlib.crc32(data)
    assert O.crc32(b"") == 0


# ---------------------------------------------------------- quantisation ---


def _group(values, g=32):
    x = np.zeros((1, g), dtype=np.float32)
    x[0, : len(values)] = values
    return x


@pytest.mark.parametrize("impl", [O.quantize_np, O.quantize_c])
def test_quantize_known_answers(impl):
    codes, scales = impl(_group([7, -7]), 4, 32)
    assert scales[0, 0] == np.float16(1.0)
    assert list(codes[0, :3]) == [15, 1, 8]
    # ties round half to even: 3.5 -> 4, 2.5 -> 2, -0.5 -> -0
    codes, _ = impl(_group([7, 3.5, 2.5, -0.5]), 4, 32)
    assert list(codes[0, :4]) == [15, 12, 10, 8]
    codes, scales = impl(np.array([[1, -1, 0.4, -0.6]], np.float32), 2, 4)
    assert list(codes[0]) == [3, 1, 2, 1] and scales[0, 0] == np.float16(1.0)
    # all-zero group: scale32 = 1e-8/7 rounds to fp16 zero, codes at the midpoint
    codes, scales = impl(np.zeros((2, 32), np.float32), 4, 32)
    assert (codes == 8).all() and (scales.view(np.uint16) == 0).all()
    codes, scales = impl(np.zeros((1, 8), np.float32), 2, 8)
    assert (codes == 2).all() and (scales.view(np.uint16) == 0).all()


@pytest.mark.parametrize("bits", [2, 4])
def test_quantize_invariants_and_implementations_agree(bits):
    rng = np.random.default_rng(bits)
    x = (rng.standard_normal((64, 8, 128)) * rng.choice([0.01, 1.0, 30.0], (64, 8, 1))).astype(np.float32)
    x[rng.random(x.shape) < 0.05] *= 8  # heavy tails
    cn, sn = O.quantize_np(x, bits, 32)
    cc, sc = O.quantize_c(x, bits, 32)
    assert np.array_equal(cn, cc) and np.array_equal(sn.view(np.uint16), sc.view(np.uint16))
    mid, top = 1 << (bits - 1), (1 << bits) - 1
    assert cn.min() >= 1 and cn.max() <= top  # raw code 0 is never produced
    groups = x.reshape(64, 8, 4, 32)
    arg = np.abs(groups).argmax(-1)
    cg = cn.reshape(64, 8, 4, 32)
    extreme = np.take_along_axis(cg, arg[..., None], -1)[..., 0].astype(int) - mid
    assert (np.abs(extreme) == mid - 1).all()  # the max-|x| element hits +-pmax
    deq = O.dequantize_np(cn, sn, bits, 32).reshape(64, 8, 4, 32)
    s32 = np.abs(groups).max(-1, keepdims=True) / (mid - 1)
    bound = s32 / 2 + (mid - 1) * s32 * 2.0**-11 + 1e-12
    assert (np.abs(deq - groups) <= bound).all()


@pytest.mark.parametrize(("bits", "max_mae"), [(4, 0.12), (2, 0.65)])
def test_quantize_round_trip_mae_like_reference(bits, max_mae):
    x = torch.randn(3, 2, 128, generator=torch.Generator().manual_seed(1)).numpy()
    codes, scales = O.quantize_c(x, bits, 32)
    restored = O.dequantize_np(codes, scales, bits, 32)
    assert np.mean(np.abs(x - restored)) < max_mae


# ------------------------------------------------------------ pack/unpack ---


def test_pack_known_answers():
    assert list(O.pack_np(np.array([1, 2], np.uint8), 4)) == [0x21]
    assert list(O.pack_np(np.array([1, 2, 3, 0], np.uint8), 2)) == [0x39]
    assert list(O.unpack_np(np.array([0x21], np.uint8), 4)) == [1, 2]
    assert list(O.unpack_np(np.array([0x39], np.uint8), 2)) == [1, 2, 3, 0]


@pytest.mark.parametrize("bits", [2, 4])
def test_pack_unpack_exhaustive(bits):
    every = np.arange(256, dtype=np.uint8)
    codes = O.unpack_np(every, bits)
    assert codes.shape == (256 * 8 // bits,)
    assert np.array_equal(O.pack_np(codes, bits), every)
    lib = O.lib()
    c_codes = np.empty_like(codes)
    lib.orc_unpack_codes(every.ctypes.data, 256, bits, c_codes.ctypes.data)
    assert np.array_equal(c_codes, codes)
    c_packed = np.empty_like(every)
    lib.orc_pack_codes(codes.ctypes.data, codes.size, bits, c_packed.ctypes.data)
    assert np.array_equal(c_packed, every)
    # low bits first: code i of a byte sits at bits [i*bits, (i+1)*bits)
    per = 8 // bits
    for i in range(per):
        assert np.array_equal(codes[i::per], (every >> (i * bits)) & ((1 << bits) - 1))


# -------------------------------------------------------------- attention ---


def make_case(seed, qh, kvh, d, nb, bt, bits, g, valid=None):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    v = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    q = rng.standard_normal((qh, d)).astype(np.float32)
    pk, sk, _ = O.quantize_blocks(k, bits, g, bt)
    pv, sv, _ = O.quantize_blocks(v, bits, g, bt)
    if valid is None:
        valid = rng.integers(1, bt + 1, nb)
    return q, pk, pv, sk, sv, np.asarray(valid, np.int32)


def dequant_tokens(pk, sk, valid, bits, g, table=None):
    nb, bt, kvh, pd = pk.shape
    d = pd * 8 // bits
    ids = range(nb) if table is None else table
    rows = []
    for b in ids:
        n = max(0, min(bt, int(valid[b])))
        codes = O.unpack_np(pk[b, :n], bits, d)
        rows.append(O.dequantize_np(codes, sk[b, :n], bits, g))
    return np.concatenate(rows, 0) if rows else np.zeros((0, kvh, d), np.float32)


@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize(("qh", "kvh", "d", "g"), [(1, 1, 32, 16), (4, 1, 64, 16), (4, 2, 128, 16), (32, 8, 128, 32)])
def test_attention_matches_torch_sdpa_float64(bits, qh, kvh, d, g):
    q, pk, pv, sk, sv, valid = make_case(41, qh, kvh, d, 3, 16, bits, g)
    scale = 1 / math.sqrt(d)
    out, lse = O.attention(q, pk, pv, sk, sv, valid, bits, g, scale)
    keys = torch.from_numpy(dequant_tokens(pk, sk, valid, bits, g)).double()
    vals = torch.from_numpy(dequant_tokens(pv, sv, valid, bits, g)).double()
    rep = qh // kvh
    kq = keys.repeat_interleave(rep, dim=1).permute(1, 0, 2)  # [QH, T, D]
    vq = vals.repeat_interleave(rep, dim=1).permute(1, 0, 2)
    qq = torch.from_numpy(q).double().unsqueeze(1)  # [QH, 1, D]
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kq, vq, scale=scale)[:, 0]
    ref_lse = torch.logsumexp((qq @ kq.transpose(1, 2))[:, 0] * scale, dim=-1)
    np.testing.assert_allclose(out, ref.numpy(), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, ref_lse.numpy(), rtol=1e-6, atol=1e-6)


def test_attention_closed_forms():
    # one token: softmax is 1, out = v, lse = s
    q, pk, pv, sk, sv, _ = make_case(3, 4, 2, 32, 2, 8, 4, 16)
    valid = np.array([1, 0], np.int32)
    out, lse = O.attention(q, pk, pv, sk, sv, valid, 4, 16, 0.25)
    kk = dequant_tokens(pk, sk, valid, 4, 16)[0]
    vv = dequant_tokens(pv, sv, valid, 4, 16)[0]
    for h in range(4):
        np.testing.assert_allclose(out[h], vv[h // 2], rtol=1e-6, atol=1e-7)
        np.testing.assert_allclose(lse[h], 0.25 * np.dot(q[h].astype(np.float64), kk[h // 2]), rtol=1e-6, atol=1e-6)
    # equal keys: uniform weights, out = mean(V), lse = s + ln T
    pk2 = np.broadcast_to(pk[:1, :1], pk.shape).copy()
    sk2 = np.broadcast_to(sk[:1, :1], sk.shape).copy()
    valid = np.array([8, 5], np.int32)
    out, lse = O.attention(q, pk2, pv, sk2, sv, valid, 4, 16, 0.25)
    vv = dequant_tokens(pv, sv, valid, 4, 16)
    kk = dequant_tokens(pk2, sk2, valid, 4, 16)[0]
    for h in range(4):
        np.testing.assert_allclose(out[h], vv[:, h // 2].mean(0), rtol=1e-5, atol=1e-6)
        s = 0.25 * np.dot(q[h].astype(np.float64), kk[h // 2])
        np.testing.assert_allclose(lse[h], s + math.log(13), rtol=1e-6, atol=1e-6)


def test_attention_brute_force_tiny():
    q, pk, pv, sk, sv, valid = make_case(9, 2, 1, 8, 2, 4, 2, 4, valid=[3, 2])
    out, lse = O.attention(q, pk, pv, sk, sv, valid, 2, 4, 0.7)
    codes_k = O.unpack_np(pk, 2)  # [2, 4, 1, 8]
    codes_v = O.unpack_np(pv, 2)
    for h in range(2):
        scores, vecs = [], []
        for b in range(2):
            for t in range(int(valid[b])):
                kd = [(int(codes_k[b, t, 0, e]) - 2) * float(sk[b, t, 0, e // 4]) for e in range(8)]
                vd = [(int(codes_v[b, t, 0, e]) - 2) * float(sv[b, t, 0, e // 4]) for e in range(8)]
                scores.append(0.7 * sum(float(q[h, e]) * kd[e] for e in range(8)))
                vecs.append(vd)
        m = max(scores)
        ws = [math.exp(s - m) for s in scores]
        tot = sum(ws)
        expect = [sum(w * v[e] for w, v in zip(ws, vecs)) / tot for e in range(8)]
        np.testing.assert_allclose(out[h], expect, rtol=1e-6, atol=1e-7)
        assert lse[h] == pytest.approx(m + math.log(tot), rel=1e-6)


def test_attention_block_table_empty_and_clamping():
    q, pk, pv, sk, sv, valid = make_case(5, 8, 2, 64, 6, 16, 4, 32)
    table = np.array([4, 1, 5], np.int32)
    out_t, lse_t = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.125, block_table=table)
    out_c, lse_c = O.attention(q, pk[table], pv[table], sk[table], sv[table], valid[table], 4, 32, 0.125)
    np.testing.assert_array_equal(out_t, out_c)
    np.testing.assert_array_equal(lse_t, lse_c)
    out, lse = O.attention(q, pk, pv, sk, sv, np.zeros(6, np.int32), 4, 32, 0.125)
    assert (out == 0).all() and np.isneginf(lse).all()
    big = np.full(6, 99, np.int32)
    o1, _ = O.attention(q, pk, pv, sk, sv, big, 4, 32, 0.125)
    o2, _ = O.attention(q, pk, pv, sk, sv, np.full(6, 16, np.int32), 4, 32, 0.125)
    np.testing.assert_array_equal(o1, o2)


def _sliced_attention(q, pk, pv, sk, sv, valid, bits, g, scale):
    """float64 attention over the rows numpy's own slice ``x[b, :valid[b]]``
    keeps: the rule of src/kvssd/backends/reference.py:38-40, applied by the
    interpreter rather than restated."""
    def deq(p, s):
        codes = O.unpack_np(p, bits, p.shape[-1] * 8 // bits).astype(np.float64) - (1 << (bits - 1))
        return codes * np.repeat(s.astype(np.float64), g, axis=-1)

    k, v = deq(pk, sk), deq(pv, sv)
    ks = np.concatenate([k[b, :n] for b, n in enumerate(valid.tolist())])
    vs = np.concatenate([v[b, :n] for b, n in enumerate(valid.tolist())])
    gq = q.shape[0] // k.shape[2]
    out = np.zeros(q.shape)
    lse = np.full(q.shape[0], -np.inf)
    for h in range(q.shape[0]):
        if len(ks) == 0:
            continue
        s = ks[:, h // gq] @ q[h].astype(np.float64) * scale
        m = s.max()
        w = np.exp(s - m)
        out[h] = w @ vs[:, h // gq] / w.sum()
        lse[h] = m + np.log(w.sum())
    return out, lse


@pytest.mark.parametrize("counts", [[16, 3, -5, 16, -16, 9], [-1, -20, 40, -15, 0, -3], [-16] * 6])
def test_attention_negative_counts_follow_the_slice_rule(counts):
    # a negative count drops rows from the end of its block, as keys[b, :v] does
    q, pk, pv, sk, sv, _ = make_case(5, 8, 2, 64, 6, 16, 4, 32)
    valid = np.array(counts, np.int32)
    out, lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.125)
    ref_out, ref_lse = _sliced_attention(q, pk, pv, sk, sv, valid, 4, 32, 0.125)
    np.testing.assert_allclose(out, ref_out, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(lse, ref_lse, rtol=1e-6, atol=1e-6)


def test_merge_split_anywhere_invariant():
    q, pk, pv, sk, sv, valid = make_case(7, 8, 2, 64, 9, 16, 4, 32)
    full, full_lse = O.attention(q, pk, pv, sk, sv, valid, 4, 32, 0.125)
    for cut in (1, 4, 8):
        a, la = O.attention(q, pk[:cut], pv[:cut], sk[:cut], sv[:cut], valid[:cut], 4, 32, 0.125)
        b, lb = O.attention(q, pk[cut:], pv[cut:], sk[cut:], sv[cut:], valid[cut:], 4, 32, 0.125)
        m, lm = O.merge(a, la, b, lb)
        np.testing.assert_allclose(m, full, rtol=1e-5, atol=1e-6)
        np.testing.assert_allclose(lm, full_lse, rtol=1e-6, atol=1e-6)
    empty_o, empty_l = np.zeros_like(full), np.full_like(full_lse, -np.inf)
    m, lm = O.merge(full, full_lse, empty_o, empty_l)
    np.testing.assert_allclose(m, full, rtol=1e-6)
    np.testing.assert_array_equal(lm, full_lse)
    m, lm = O.merge(empty_o, empty_l, empty_o, empty_l)
    assert (m == 0).all() and np.isneginf(lm).all()


# -------------------------------------------------------------- selectors ---


def test_selector_known_answers():
    assert O.select_recent_sink(list(range(2048)), 1, 32) == [0] + list(range(2016, 2048))
    assert O.select_recent_sink([0, 1, 2], 1, 0) == [0]
    assert O.select_recent_sink([0, 1, 2], 2, 2) == [0, 1, 2]
    assert O.select_recent_sink([5, 9], 3, 3) == [5, 9]
    assert O.select_recent_sink([5, 9], 0, 3) == [5, 9]
    assert O.select_recent_sink([4, 5, 9], 1, 1) == [4, 9]
    assert O.select_all([3, 1, 2]) == [3, 1, 2]
    with pytest.raises(ValueError):
        O.select_recent_sink([0], -1, 0)


# ----------------------------------------------------------------- record ---


def test_record_layout_known_answers():
    assert O.HEADER.size == 52
    assert O.record_bytes(8, 128, 128, 4, 32) == 151552
    assert O.record_bytes(8, 128, 128, 2, 32) == 86016
    ks = np.arange(2 * 1 * 2, dtype=np.float16).reshape(2, 1, 2)
    kp = np.arange(2 * 1 * 8, dtype=np.uint8).reshape(2, 1, 8)
    rec = O.encode_record(3, 7, 2, 4, 2, 1, 16, 8, ks, ks, kp, kp)
    assert len(rec) == 4096
    fields = struct.unpack("<8sIIIIIIIIIII", rec[:52])
    assert fields[:11] == (b"KVSSD001", 1, 3, 7, 2, 4, 2, 1, 16, 8, 2 * 8 + 2 * 16)
    payload = rec[52 : 52 + fields[10]]
    assert fields[11] == zlib.crc32(payload)
    assert payload[:8] == ks.tobytes() and payload[16:32] == kp.tobytes()
    assert rec[52 + fields[10] :] == bytes(4096 - 52 - fields[10])


# ------------------------------------------------------------- vLLM block ---


def test_vllm_record_known_answer():
    # [7, -7, 0, 0] with g=4, INT4: scale 7/7 = 1.0 (fp16 0x3C00), codes
    # [15, 1, 8, 8] -> packed low nibble first [0x1F, 0x88]
    rec = O.encode_vllm_record(np.array([7.0, -7.0, 0.0, 0.0]), 4, 4, 1)
    payload = bytes([0x00, 0x3C, 0x1F, 0x88])
    head = struct.pack("<8sBBBBIIQI", b"KVVLLM02", 1, 4, 1, 0, 4, 4, 4, zlib.crc32(payload))
    assert len(rec) == 4096
    assert rec[:32] == head and rec[32:36] == payload and rec[36:] == bytes(4096 - 36)
    assert O.decode_vllm_values(rec).tolist() == [7.0, -7.0, 0.0, 0.0]
    # INT2, g=4: [1, -1, 0.4, -0.6] -> scale 1.0, codes [3, 1, 2, 1] -> 0b01_10_01_11
    rec2 = O.encode_vllm_record(np.array([1.0, -1.0, 0.4, -0.6]), 2, 4, 3)
    assert rec2[32:35] == bytes([0x00, 0x3C, 0x67])
    assert struct.unpack_from("<8sBBBBIIQI", rec2)[7] == 3
    assert O.decode_vllm_values(rec2).tolist() == [1.0, -1.0, 0.0, -1.0]


def test_vllm_record_round_trip_bound():
    rng = np.random.default_rng(9)
    x = rng.standard_normal(4096).astype(np.float32)
    rec = O.encode_vllm_record(x, 4, 32, 3)
    y = O.decode_vllm_values(rec)
    step = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True) / 7
    assert np.all(np.abs((y - x).reshape(-1, 32)) <= step * 0.5 + 1e-3 * step)
