"""The HIP kernels on the committed golden fixtures (tests/golden/*.npz),
through the C ABI: decode outputs within max-abs 2e-3 / rel 1e-2 for every
kernel that takes the shape, unpacked codes bit for bit."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from kvssd import _native
from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))
import make_golden  # noqa: E402

ATOL, RTOL = 2e-3, 1e-2


def load(name: str) -> dict[str, np.ndarray]:
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


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


@pytest.mark.parametrize("name", [c[0] for c in make_golden.DECODE_CASES])
def test_kernels_on_decode_fixture(cuda_device, name):
    fix = load(name)
    query = torch.from_numpy(fix["q"]).to(torch.float16).to(cuda_device)
    batch = PackedBatch(*(torch.from_numpy(fix[k]).to(cuda_device)
                          for k in ("packed_k", "packed_v", "scales_k", "scales_v", "valid")),
                        int(fix["bits"]), int(fix["group_size"]))
    for kernel in kernels_for(query, batch):
        backend = HipAttentionBackend(kernel)
        out, lse = backend.run(query, batch, float(fix["sm_scale"]))
        assert backend.last_kernel == kernel
        np.testing.assert_allclose(out.cpu().numpy(), fix["out"], atol=ATOL, rtol=RTOL, err_msg=kernel)
        np.testing.assert_allclose(lse.cpu().numpy(), fix["lse"], atol=ATOL, rtol=RTOL, err_msg=kernel)


@pytest.mark.parametrize("bits", [2, 4])
def test_unpack_kernel_on_codec_fixture(cuda_device, bits):
    fix = load("codec")
    packed = torch.from_numpy(fix[f"packed{bits}"]).contiguous().to(cuda_device)
    codes = torch.full((packed.numel() * 8 // bits,), 255, dtype=torch.uint8, device=cuda_device)
    rc = _native.load().kvssd_hip_unpack_codes(packed.data_ptr(), bits, packed.numel(), codes.data_ptr(), None)
    _native.check(rc, "unpack")
    torch.cuda.synchronize()
    assert np.array_equal(codes.cpu().numpy().reshape(fix[f"codes{bits}"].shape), fix[f"codes{bits}"])
