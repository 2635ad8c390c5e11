"""Write the golden fixtures of tests/golden/ from the CPU oracle.

    python tests/golden/make_golden.py

Each case is a small seeded input and the oracle's output for it, saved as a
.npz (plain arrays, no pickles).  tests/test_golden.py re-derives every case on
the CPU and checks it bit for bit (integer data) or to the last float bits
(attention), so a change to the oracle or to the package's quantiser shows up
as a fixture mismatch; tests/test_gpu_golden.py runs the HIP kernels on the
same inputs.  The reference ships no golden vectors of its own for this path.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT))

from oracle import oracle as O  # noqa: E402

# (name, seed, query heads, kv heads, head dim, group, blocks, block tokens, bits, valid)
DECODE_CASES = [
    ("decode_int4_gqa4", 101, 8, 2, 128, 32, 3, 128, 4, [128, 77, 1]),
    ("decode_int2_gqa4", 102, 8, 2, 128, 32, 3, 128, 2, [128, 128, 5]),
    ("decode_int4_kvh4", 103, 16, 4, 128, 32, 2, 128, 4, [100, 128]),
    ("decode_int4_ref_shape", 104, 4, 2, 128, 16, 2, 8, 4, [8, 5]),
    ("decode_int2_ref_shape", 105, 4, 1, 64, 16, 2, 8, 2, [8, 5]),
]


def decode_case(seed, qh, kvh, d, g, nb, bt, bits, valid):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    v = rng.standard_normal((nb * bt, kvh, d)).astype(np.float32)
    q = rng.standard_normal((qh, d)).astype(np.float16).astype(np.float32)
    pk, sk, _ = O.quantize_blocks(k, bits, g, bt)
    pv, sv, _ = O.quantize_blocks(v, bits, g, bt)
    valid = np.asarray(valid, np.int32)
    scale = 1.0 / np.sqrt(d)
    out, lse = O.attention(q, pk, pv, sk, sv, valid, bits, g, scale)
    return dict(q=q, packed_k=pk, packed_v=pv, scales_k=sk, scales_v=sv, valid=valid,
                bits=np.int32(bits), group_size=np.int32(g), sm_scale=np.float64(scale), out=out, lse=lse)


def codec_case():
    rng = np.random.default_rng(201)
    x = (rng.standard_normal((64, 128)) * rng.choice([1e-3, 1.0, 50.0], (64, 1))).astype(np.float32)
    x[3] = 0.0  # an all-zero row: scale 0, codes = mid
    res = {"x": x}
    for bits in (2, 4):
        codes, scales = O.quantize_c(x, bits, 32)
        res[f"codes{bits}"] = codes
        res[f"scales{bits}"] = scales.view(np.uint16)
        res[f"packed{bits}"] = O.pack_np(codes, bits)
    return res


def selection_case():
    avail = list(range(2048))
    return {
        "recent_sink_1_32": np.asarray(O.select_recent_sink(avail, 1, 32), np.int32),
        "recent_sink_2_3": np.asarray(O.select_recent_sink(avail, 2, 3), np.int32),
        "recent_sink_0_1": np.asarray(O.select_recent_sink(avail, 0, 1), np.int32),
        "all_32": np.asarray(O.select_all(list(range(32))), np.int32),
    }


def build_all() -> dict[str, dict[str, np.ndarray]]:
    cases = {name: decode_case(*args) for name, *args in DECODE_CASES}
    cases["codec"] = codec_case()
    cases["selection"] = selection_case()
    return cases


def main() -> None:
    for name, arrays in build_all().items():
        np.savez_compressed(HERE / f"{name}.npz", **arrays)
        print(name, sum(a.nbytes for a in arrays.values()), "bytes")


if __name__ == "__main__":
    main()
