"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the CPU oracle) against a fresh oracle run and
against the package's own CPU code: quantiser, packer, selectors and the
reference backend.  Integer data must match bit for bit."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd.backends import PackedBatch
from kvssd.backends.reference import ReferenceAttentionBackend
from kvssd.quant import pack_codes, quantize_tensor, unpack_codes
from kvssd.selectors import AllBlocks, RecentSinkBlocks

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden  # noqa: E402

DECODE = [c[0] for c in make_golden.DECODE_CASES]


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.mark.parametrize("name", DECODE)
def test_oracle_reproduces_decode_fixture(name):
    args = next(c[1:] for c in make_golden.DECODE_CASES if c[0] == name)
    fresh = make_golden.decode_case(*args)
    fix = load(name)
    for key in ("q", "packed_k", "packed_v", "scales_k", "scales_v", "valid"):
        assert np.array_equal(fresh[key], fix[key]), key
    np.testing.assert_allclose(fresh["out"], fix["out"], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(fresh["lse"], fix["lse"], rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("name", DECODE)
def test_reference_backend_on_decode_fixture(name):
    fix = load(name)
    batch = PackedBatch(*(torch.from_numpy(fix[k]) for k in ("packed_k", "packed_v", "scales_k", "scales_v", "valid")),
                        int(fix["bits"]), int(fix["group_size"]))
    out, lse = ReferenceAttentionBackend().run(torch.from_numpy(fix["q"]), batch, float(fix["sm_scale"]))
    np.testing.assert_allclose(out.numpy(), fix["out"], atol=2e-5, rtol=1e-5)
    np.testing.assert_allclose(lse.numpy(), fix["lse"], atol=2e-5, rtol=1e-5)


def test_codec_fixture_bit_exact():
    fix = load("codec")
    fresh = make_golden.codec_case()
    x = torch.from_numpy(fix["x"])
    for bits in (2, 4):
        assert np.array_equal(fresh[f"codes{bits}"], fix[f"codes{bits}"])
        assert np.array_equal(fresh[f"scales{bits}"], fix[f"scales{bits}"])
        assert np.array_equal(fresh[f"packed{bits}"], fix[f"packed{bits}"])
        q = quantize_tensor(x, bits, 32)
        assert np.array_equal(q.packed.numpy(), fix[f"packed{bits}"])
        assert np.array_equal(q.scales.numpy().view(np.uint16), fix[f"scales{bits}"])
        codes = torch.from_numpy(fix[f"codes{bits}"])
        assert np.array_equal(pack_codes(codes, bits).numpy(), fix[f"packed{bits}"])
        unpacked = unpack_codes(torch.from_numpy(fix[f"packed{bits}"]), bits, codes.shape[-1])
        assert np.array_equal(unpacked.numpy(), fix[f"codes{bits}"])


def test_selection_fixture():
    fix = load("selection")
    avail = list(range(2048))
    assert RecentSinkBlocks(1, 32).select(avail) == fix["recent_sink_1_32"].tolist()
    assert RecentSinkBlocks(2, 3).select(avail) == fix["recent_sink_2_3"].tolist()
    assert RecentSinkBlocks(0, 1).select(avail) == fix["recent_sink_0_1"].tolist()
    assert AllBlocks().select(list(range(32))) == fix["all_32"].tolist()
    assert fix["recent_sink_1_32"].tolist() == [0] + list(range(2016, 2048))
