"""The streaming-read probe behind bench.py's ``roofline.attainable`` reads
every byte it is given: the XOR of its sink equals the XOR of every dword of
the data (each 16-byte chunk lands in one lane, each lane in one wave's
dword), for sizes that leave every tail of the unrolled loop in use."""

import numpy as np
import pytest
import torch

from kvssd import _native

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes", [16, 4096, 16 * 2048 * 256 * 4 + 48, 3 << 20])
def test_read_probe_folds_every_dword(cuda_device, nbytes):
    lib = _native.load()
    rng = np.random.default_rng(nbytes)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    data = torch.from_numpy(host.view(np.int32)).to(cuda_device)
    sink = torch.full((8192,), -1, dtype=torch.int32, device=cuda_device)
    sh = _native.stream_handle(torch.cuda.current_stream(cuda_device))
    _native.check(lib.kvssd_hip_read_probe(data.data_ptr(), nbytes, sink.data_ptr(), sink.numel(), sh), "probe")
    got = np.bitwise_xor.reduce(sink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)
