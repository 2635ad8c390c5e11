"""The needle design of tests/needles.py, checked on the CPU with the oracle:
the needles carry the softmax mass, the check accepts the oracle against
itself, and it rejects the oracle with one block, one 32-token segment or one
needle removed.  The GPU tests rely on exactly these properties at full size."""

from __future__ import annotations

import numpy as np
import pytest

import needles as N


@pytest.mark.parametrize(("bits", "outliers", "target"), [(4, 0.0, 10.0), (2, 0.05, 16.0)])
def test_needle_check_sees_one_missing_block_segment_or_needle(bits, outliers, target):
    nb = 96
    q16, k, v = N.half_kv(nb * 128, 3 + bits, 1.0, outliers, 32)
    rng = np.random.default_rng(bits)
    valid = np.full(nb, 128, np.int32)
    valid[5] = 77
    valid[9] = 0
    needles = N.plant(k.reshape(nb, 128, 8, 128), v.reshape(nb, 128, 8, 128), q16.float().numpy(), valid,
                      N.SCALE, rng, amp=128.0, target=target)
    arrays, _ = N.quantize(k, v, bits)
    q = q16.float().numpy()
    ref_out, ref_lse = N.oracle(q, arrays, valid, bits)
    assert N.needle_mass_share(q, arrays[0], arrays[2], bits, needles, ref_lse) > 0.98
    N.assert_sensitive_match(ref_out, ref_lse, ref_out, ref_lse)
    ctl = N.controls(q, arrays, valid, bits, None, needles)
    assert set(ctl) == {"block", "segment", "needle"}
    for name, (c_out, c_lse) in ctl.items():
        assert N.differs(ref_out, ref_lse, c_out, c_lse), name
        with pytest.raises(AssertionError):
            N.assert_sensitive_match(c_out, c_lse, ref_out, ref_lse, name)


def test_needle_rows_cover_every_segment_of_the_attended_rows():
    rng = np.random.default_rng(0)
    valid = np.array([128, 0, 33, -96, 200], np.int32)
    bb, tt = N.needle_rows(valid, 128, rng)
    for b, rows in ((0, 128), (1, 0), (2, 33), (3, 32), (4, 128)):
        got = sorted(tt[bb == b].tolist())
        assert all(0 <= r < rows for r in got)
        for s0 in range(0, rows, 32):
            seg = [r for r in got if s0 <= r < min(rows, s0 + 32)]
            assert s0 in seg and min(rows, s0 + 32) - 1 in seg
            assert len(seg) == min(4, min(rows, s0 + 32) - s0)


def test_moving_rows_to_the_end_removes_exactly_those_rows():
    q16, k, v = N.half_kv(8 * 128, 1, 1.0, 0.0, 32)
    arrays, valid = N.quantize(k, v, 4)
    q = q16.float().numpy()
    drop = [3, 64, 100]
    moved = N.move_rows_to_end(arrays, 2, drop)
    v2 = valid.copy()
    v2[2] -= len(drop)
    out, lse = N.oracle(q, moved, v2, 4)
    # the same rows removed by building the block without them
    keep = [r for r in range(128) if r not in drop]
    pk, pv, sk, sv = (a.copy() for a in arrays)
    for a, src in zip((pk, pv, sk, sv), arrays):
        a[2, : len(keep)] = src[2, keep]
    out2, lse2 = N.oracle(q, [pk, pv, sk, sv], v2, 4)
    np.testing.assert_array_equal(out, out2)
    np.testing.assert_array_equal(lse, lse2)


def test_segment_runs_share_dim_and_sign():
    rng = np.random.default_rng(5)
    v = N.needle_values(10, 3, 16, 8.0, rng, run=4)
    nz = [np.flatnonzero(v[i, 1]) for i in range(10)]
    assert all(len(x) == 1 for x in nz)
    for a, b in ((0, 3), (4, 7), (8, 9)):
        assert nz[a][0] == nz[b][0] and v[a, 1, nz[a][0]] == v[b, 1, nz[b][0]]
