"""kvssd_hip_fused_decode_static, the decode that allocates nothing (its split
partials live in the library's per-GPU static scratch), against
kvssd_hip_fused_decode with a caller's workspace: bit-identical results on two
calls in a row, the second over a smaller input, both through the C ABI; the
first also against the CPU oracle at the contract tolerance."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

from kvssd import _native
from kvssd.backends import PackedBatch
from kvssd.backends.hip import HipAttentionBackend
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _inputs(dev, seed, nb, bits=4, qh=32, kvh=8):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nb * 128, kvh, 128)).astype(np.float32)
    v = rng.standard_normal((nb * 128, kvh, 128)).astype(np.float32)
    q = rng.standard_normal((qh, 128)).astype(np.float32)
    pk, sk, valid = O.quantize_blocks(k, bits, 32, 128)
    pv, sv, _ = O.quantize_blocks(v, bits, 32, 128)
    valid[nb // 3] = 77
    host = (pk, pv, sk, sv, valid)
    batch = PackedBatch(*(torch.from_numpy(a).to(dev) for a in host), bits, 32)
    query = torch.from_numpy(q).to(torch.float16).to(dev)
    return query, batch, host


def _both(dev, query, batch):
    lib = _native.load()
    scale = 1 / math.sqrt(128)
    desc = HipAttentionBackend().describe(query, batch, scale)
    need = ctypes.c_size_t(0)
    _native.check(lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(need)), "workspace")
    work = torch.empty(int(need.value), dtype=torch.uint8, device=dev)
    stream = _native.stream_handle(torch.cuda.current_stream(dev))
    ptrs = (query.data_ptr(), batch.packed_k.data_ptr(), batch.packed_v.data_ptr(), batch.scales_k.data_ptr(),
            batch.scales_v.data_ptr(), batch.valid_tokens.data_ptr(), None)
    qh = query.shape[0]
    out_ws = torch.full((qh, 128), float("nan"), device=dev)
    lse_ws = torch.full((qh,), float("nan"), device=dev)
    out_st = torch.full((qh, 128), float("nan"), device=dev)
    lse_st = torch.full((qh,), float("nan"), device=dev)
    _native.check(lib.kvssd_hip_fused_decode(ctypes.byref(desc), *ptrs, out_ws.data_ptr(), lse_ws.data_ptr(),
                                             work.data_ptr(), work.numel(), stream), "fused_decode")
    _native.check(lib.kvssd_hip_fused_decode_static(ctypes.byref(desc), *ptrs, out_st.data_ptr(), lse_st.data_ptr(),
                                                    stream), "fused_decode_static")
    torch.cuda.synchronize()
    return (out_ws, lse_ws), (out_st, lse_st), int(need.value)


def test_static_scratch_decode_matches_the_workspace_decode(cuda_device):
    first = None
    for seed, nb in ((1, 1024), (2, 37)):  # 128K tokens, then a smaller input
        query, batch, host = _inputs(cuda_device, seed, nb)
        (o_ws, l_ws), (o_st, l_st), need = _both(cuda_device, query, batch)
        assert need <= 16 << 20
        assert torch.equal(o_st, o_ws) and torch.equal(l_st, l_ws), f"{nb} blocks: static scratch differs"
        if first is None:
            first = nb
            ref_out, ref_lse = O.attention(query.float().cpu().numpy(), *host, 4, 32, 1 / math.sqrt(128), threads=16)
            np.testing.assert_allclose(o_st.cpu().numpy(), ref_out, atol=2e-3, rtol=1e-2)
            np.testing.assert_allclose(l_st.cpu().numpy(), ref_lse, atol=2e-3, rtol=1e-2)
