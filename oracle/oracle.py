"""CPU oracle for the fused INT2/INT4 decode-attention path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s cpu_baseline leg import this module, and only to check results.
The ``kvssd`` package never imports it.

It restates the reference algorithm from its source (citations per function):
numpy for byte/integer arithmetic and the record format, and the plain-C
library ``oracle/_build/libkvssd_oracle.so`` (built from ``kvssd_oracle.c`` by
``oracle/Makefile``) for the dequantise-then-attend computation, which it runs
with double-precision accumulation.

How each function is pinned is listed in ``tests/test_oracle.py``; nothing here
is "parity unpinned".
"""

from __future__ import annotations

import ctypes
import os
import struct
import subprocess
import zlib
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkvssd_oracle.so"

# Record layout restated from src/kvssd/format.py:14-16 (constants) and :104-131 (the encoder).
ALIGNMENT = 4096
MAGIC = b"KVSSD001"
HEADER = struct.Struct("<8sIIIIIIIIIII")

_lib = None


def build() -> Path:
    """Compile the C oracle with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        handle = ctypes.CDLL(str(LIB_PATH))
        c = ctypes
        handle.orc_f16_to_f32.restype = c.c_float
        handle.orc_f16_to_f32.argtypes = [c.c_uint16]
        handle.orc_f32_to_f16.restype = c.c_uint16
        handle.orc_f32_to_f16.argtypes = [c.c_float]
        handle.orc_quantize_groups.restype = None
        handle.orc_quantize_groups.argtypes = [c.c_void_p, c.c_int64, c.c_int, c.c_int, c.c_void_p, c.c_void_p]
        handle.orc_pack_codes.restype = None
        handle.orc_pack_codes.argtypes = [c.c_void_p, c.c_int64, c.c_int, c.c_void_p]
        handle.orc_unpack_codes.restype = None
        handle.orc_unpack_codes.argtypes = [c.c_void_p, c.c_int64, c.c_int, c.c_void_p]
        handle.orc_decode_attention.restype = c.c_int
        handle.orc_decode_attention.argtypes = [c.c_int] * 7 + [c.c_void_p] * 7 + [
            c.c_int,
            c.c_double,
            c.c_void_p,
            c.c_void_p,
            c.c_int,
        ]
        handle.orc_merge.restype = None
        handle.orc_merge.argtypes = [c.c_int, c.c_int] + [c.c_void_p] * 6
        handle.orc_crc32.restype = c.c_uint32
        handle.orc_crc32.argtypes = [c.c_void_p, c.c_size_t, c.c_uint32]
        _lib = handle
    return _lib


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


# ----------------------------------------------------------------- numpy ---


def quantize_np(x: np.ndarray, bits: int, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Unpacked codes (uint8, x.shape) and fp16 scales ([..., D/g]).

    Restates src/kvssd/quant.py:49-65 with numpy float32 arithmetic: IEEE
    division, ``np.rint`` (round half to even, as ``torch.round``), then
    ``astype(float16)`` (round to nearest even) for the stored scale.
    """
    x = np.ascontiguousarray(x, dtype=np.float32)
    mid = 1 << (bits - 1)
    pmax = np.float32(mid - 1)
    groups = x.reshape(*x.shape[:-1], x.shape[-1] // group_size, group_size)
    amax = np.abs(groups).max(axis=-1)
    scale32 = np.maximum(amax, np.float32(1e-8)).astype(np.float32) / pmax
    ratio = (groups / scale32[..., None]).astype(np.float32)
    codes = np.clip(np.rint(ratio), -mid, mid - 1) + mid
    return codes.astype(np.uint8).reshape(x.shape), scale32.astype(np.float16)


def quantize_c(x: np.ndarray, bits: int, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Same contract as :func:`quantize_np`, computed by the C oracle."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n_groups = x.size // group_size
    codes = np.empty(x.shape, dtype=np.uint8)
    scales = np.empty((*x.shape[:-1], x.shape[-1] // group_size), dtype=np.uint16)
    lib().orc_quantize_groups(_ptr(x), n_groups, group_size, bits, _ptr(codes), _ptr(scales))
    return codes, scales.view(np.float16)


def pack_np(codes: np.ndarray, bits: int) -> np.ndarray:
    """Low-bits-first packing along the last dim (src/kvssd/quant.py:28-37)."""
    per = 8 // bits
    c = codes.astype(np.uint16).reshape(*codes.shape[:-1], -1, per)
    out = np.zeros(c.shape[:-1], dtype=np.uint16)
    for i in range(per):
        out |= (c[..., i] & ((1 << bits) - 1)) << (i * bits)
    return out.astype(np.uint8)


def unpack_np(packed: np.ndarray, bits: int, elements: int | None = None) -> np.ndarray:
    """Inverse of :func:`pack_np`, as unpack_codes (src/kvssd/quant.py:40-46)."""
    per = 8 // bits
    shifts = np.arange(per, dtype=np.uint8) * bits
    vals = (packed[..., None] >> shifts) & ((1 << bits) - 1)
    vals = vals.reshape(*packed.shape[:-1], packed.shape[-1] * per).astype(np.uint8)
    return vals if elements is None else vals[..., :elements]


def dequantize_np(codes: np.ndarray, scales: np.ndarray, bits: int, group_size: int) -> np.ndarray:
    """(code - mid) * scale in float32 (src/kvssd/quant.py:68-73); exact."""
    mid = 1 << (bits - 1)
    g = codes.astype(np.float32).reshape(*codes.shape[:-1], codes.shape[-1] // group_size, group_size) - mid
    return (g * scales.astype(np.float32)[..., None]).reshape(codes.shape)


def quantize_blocks(x: np.ndarray, bits: int, group_size: int, block_tokens: int):
    """Pad [T, KVH, D] to whole blocks and quantise, as KVCacheStore.create does
    per block (src/kvssd/store.py:46-60).  Quantisation groups lie along the last
    dim only, so quantising the padded tensor at once gives the same bytes.
    Returns (packed [NB, BT, KVH, PD] u8, scales [NB, BT, KVH, G] f16, valid i32)."""
    t, kvh, d = x.shape
    nb = -(-t // block_tokens)
    padded = np.zeros((nb * block_tokens, kvh, d), dtype=np.float32)
    padded[:t] = x
    codes, scales = quantize_c(padded, bits, group_size)
    packed = pack_np(codes, bits).reshape(nb, block_tokens, kvh, d * bits // 8)
    valid = np.array([min(block_tokens, t - i * block_tokens) for i in range(nb)], dtype=np.int32)
    return packed, scales.reshape(nb, block_tokens, kvh, d // group_size), valid


# ------------------------------------------------------------- selectors ---


def select_all(available: list[int]) -> list[int]:
    """AllBlocks.select (src/kvssd/selectors.py:11-14)."""
    return list(available)


def select_recent_sink(available: list[int], sink: int, recent: int) -> list[int]:
    """RecentSinkBlocks.select (src/kvssd/selectors.py:17-28): the first
    ``sink`` and last ``recent`` ids, order kept, first occurrence wins."""
    if sink < 0 or recent < 0:
        raise ValueError("sink and recent counts must be non-negative")
    head = available[:sink]
    tail = available[max(0, len(available) - recent) :] if recent else []
    out: list[int] = []
    seen: set[int] = set()
    for item in head + tail:
        if item not in seen:
            seen.add(item)
            out.append(item)
    return out


# ----------------------------------------------------------------- record ---


def record_bytes(kv_heads: int, head_dim: int, block_tokens: int, bits: int, group_size: int) -> int:
    """CacheSpec.record_bytes (src/kvssd/format.py:53-58)."""
    scale_count = block_tokens * kv_heads * (head_dim // group_size)
    packed_count = block_tokens * kv_heads * head_dim * bits // 8
    payload = 2 * scale_count * 2 + 2 * packed_count
    return -(-(HEADER.size + payload) // ALIGNMENT) * ALIGNMENT


def encode_record(layer, block, valid, bits, block_tokens, kv_heads, head_dim, group_size, ks, vs, kp, vp) -> bytes:
    """Record v1 (src/kvssd/format.py:104-131): 52-byte header, payload
    Ks | Vs | Kc | Vc, zero padding to a 4096 multiple; CRC-32 of the payload."""
    payload = b"".join(
        np.ascontiguousarray(a).tobytes()
        for a in (ks.astype(np.float16), vs.astype(np.float16), kp.astype(np.uint8), vp.astype(np.uint8))
    )
    crc = crc32(payload)
    head = HEADER.pack(
        MAGIC, 1, layer, block, valid, bits, block_tokens, kv_heads, head_dim, group_size, len(payload), crc
    )
    rec = head + payload
    total = record_bytes(kv_heads, head_dim, block_tokens, bits, group_size)
    return rec + bytes(total - len(rec))


def crc32(data: bytes, init: int = 0) -> int:
    """CRC-32 by the C oracle (pinned to zlib.crc32 and the standard check value)."""
    buf = np.frombuffer(data, dtype=np.uint8)
    buf = np.ascontiguousarray(buf)
    return int(lib().orc_crc32(_ptr(buf), buf.size, init))


def crc32_zlib(data: bytes) -> int:
    return zlib.crc32(data)


# ------------------------------------------------------------ vLLM block ---

# Restated from src/kvssd/integrations/vllm_codec.py:18-21.
VLLM_MAGIC = b"KVVLLM02"
VLLM_HEADER = struct.Struct("<8sBBBBIIQI")


def encode_vllm_record(values: np.ndarray, bits: int, group_size: int, dtype_code: int) -> bytes:
    """encode_vllm_block (src/kvssd/integrations/vllm_codec.py:42-70): the block's
    values as one flat vector quantised groupwise; payload = fp16 scales | packed
    codes; 32-byte header; zero padding to a 4096 multiple.  ``values`` are the
    block's values converted to float32 (quantize_tensor works on x.float())."""
    flat = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    codes, scales = quantize_np(flat, bits, group_size)
    payload = scales.astype(np.float16).tobytes() + pack_np(codes, bits).tobytes()
    head = VLLM_HEADER.pack(VLLM_MAGIC, 1, bits, dtype_code, 0, group_size, flat.size, len(payload), crc32(payload))
    rec = head + payload
    return rec + bytes(-(-len(rec) // ALIGNMENT) * ALIGNMENT - len(rec))


def decode_vllm_values(record: bytes) -> np.ndarray:
    """The float32 values decode_vllm_block dequantises (vllm_codec.py:73-102,
    before the cast to the record's dtype): (code - mid) * scale per group."""
    _, _, bits, _, _, g, elements, plen, _ = VLLM_HEADER.unpack_from(record)
    payload = record[VLLM_HEADER.size : VLLM_HEADER.size + plen]
    nscale = elements // g
    scales = np.frombuffer(payload[: 2 * nscale], dtype=np.float16)
    codes = unpack_np(np.frombuffer(payload[2 * nscale :], dtype=np.uint8), bits, elements)
    return dequantize_np(codes, scales, bits, g)


# -------------------------------------------------------------- attention ---


def attention(
    query: np.ndarray,
    packed_k: np.ndarray,
    packed_v: np.ndarray,
    scales_k: np.ndarray,
    scales_v: np.ndarray,
    valid: np.ndarray,
    bits: int,
    group_size: int,
    sm_scale: float,
    block_table: np.ndarray | None = None,
    threads: int = 0,
) -> tuple[np.ndarray, np.ndarray]:
    """(out fp32 [QH, D], lse fp32 [QH]) of ReferenceAttentionBackend.run
    (src/kvssd/backends/reference.py:22-50), by the C oracle."""
    q = np.ascontiguousarray(query, dtype=np.float32)
    qh, d = q.shape
    nb, bt, kvh, _pd = packed_k.shape
    pk = np.ascontiguousarray(packed_k, dtype=np.uint8)
    pv = np.ascontiguousarray(packed_v, dtype=np.uint8)
    sk = np.ascontiguousarray(scales_k.astype(np.float16)).view(np.uint16)
    sv = np.ascontiguousarray(scales_v.astype(np.float16)).view(np.uint16)
    va = np.ascontiguousarray(valid, dtype=np.int32)
    bt_arr = None if block_table is None else np.ascontiguousarray(block_table, dtype=np.int32)
    out = np.empty((qh, d), dtype=np.float32)
    lse = np.empty((qh,), dtype=np.float32)
    rc = lib().orc_decode_attention(
        qh,
        kvh,
        d,
        nb,
        bt,
        bits,
        group_size,
        _ptr(q),
        _ptr(pk),
        _ptr(pv),
        _ptr(sk),
        _ptr(sv),
        _ptr(va),
        _ptr(bt_arr),
        0 if bt_arr is None else int(bt_arr.size),
        float(sm_scale),
        _ptr(out),
        _ptr(lse),
        int(threads),
    )
    if rc != 0:
        raise ValueError("oracle rejected the attention shapes")
    return out, lse


def merge(oa: np.ndarray, la: np.ndarray, ob: np.ndarray, lb: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """merge_attention_chunks (src/kvssd/attention.py:91-102) by the C oracle."""
    oa = np.ascontiguousarray(oa, dtype=np.float32)
    ob = np.ascontiguousarray(ob, dtype=np.float32)
    la = np.ascontiguousarray(la, dtype=np.float32)
    lb = np.ascontiguousarray(lb, dtype=np.float32)
    rows, d = oa.shape
    out = np.empty_like(oa)
    lout = np.empty_like(la)
    lib().orc_merge(rows, d, _ptr(oa), _ptr(la), _ptr(ob), _ptr(lb), _ptr(out), _ptr(lout))
    return out, lout


def cpu_count() -> int:
    """Threads for the oracle: OMP_NUM_THREADS when set (the host's CPU share),
    else the usable cores, at most 16."""
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit() and int(env) > 0:
        return int(env)
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        usable = os.cpu_count() or 1
    return max(1, min(16, usable))
