"""Per-workgroup phase timeline of one decode, from the instrumented library.

    python kvssd-attention_amd/csrc/build.py --timeline        # once, on any host with hipcc
    python kvssd-attention_amd/csrc/timeline.py [--workload int4_gqa_128k] [--calls 3]

The instrumented build (csrc/timeline.hpp) stamps the 100 MHz real-time clock
when each workgroup's wave 0 passes a phase: entry, the stage loop, every stage
barrier, the end of the loop and the partial stores (the prologue's copies in
between).  It runs the
bench workload's decode (after a warm-up, back to back with the call before)
in a child process that loads only that build, and prints each phase's
min / median / max over the workgroups, in microseconds from the first
workgroup's entry (the split kernel; the merge kernel is not instrumented),
the median end of the stage loop by XCD, and how well a workgroup's end time
in one call predicts it in the next.
"""

from __future__ import annotations

import argparse
import ctypes
import math
import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
LIB = HERE.parent / "kvssd" / "libkvssd_hip_timeline.so"
SLOTS = 64
WGS = 4096
NAMES = {0: "entry", 22: "st0 issued", 23: "rows landed", 24: "st1 issued", 25: "st0 landed", 1: "loop",
         18: "loop end", 19: "stored"}
for k in range(16):
    NAMES[2 + k] = f"stage {k}" if k < 15 else "stage 15+"


def child(args) -> int:
    for p in (ROOT / "kvssd-attention_amd", ROOT):
        sys.path.insert(0, str(p))
    import numpy as np
    import torch

    import bench
    from kvssd import _native
    from kvssd.backends import PackedBatch
    from kvssd.backends.hip import HipAttentionBackend

    dev = torch.device("cuda", 0)
    tokens, bits, qh, vscale, outl, sel = bench.WORKLOADS[args.workload]
    query, cache, valid = bench.make_cache(torch, dev, tokens, bits, qh, vscale, outl)
    batch = PackedBatch(cache["pk"], cache["pv"], cache["sk"], cache["sv"], valid, bits, bench.GROUP)
    copies = [batch] + [PackedBatch(*(t.clone() for t in (cache["pk"], cache["pv"], cache["sk"], cache["sv"])),
                                    valid, bits, bench.GROUP) for _ in range(3)]
    lib = _native.load()
    assert _native.LIB_PATH == LIB.resolve(), "the timeline needs the instrumented build"
    lib.kvssd_hip_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    backend = HipAttentionBackend()
    scale = 1 / math.sqrt(128)
    table = None
    if sel is not None:
        from kvssd.selectors import RecentSinkBlocks

        table = torch.tensor(RecentSinkBlocks(*sel).select(list(range(tokens // 128))), dtype=torch.int32, device=dev)
    for i in range(200):
        backend.run(query, copies[i % 4], scale, block_table=table)
    torch.cuda.synchronize()
    buf = np.zeros(WGS * SLOTS, np.uint64)
    ends = []
    for rep in range(args.calls):
        assert lib.kvssd_hip_timeline_clear() == 0
        torch.cuda.synchronize()
        backend.run(query, copies[rep % 4], scale, block_table=table)  # queued behind the previous one
        backend.run(query, copies[(rep + 1) % 4], scale, block_table=table)
        torch.cuda.synchronize()
        assert lib.kvssd_hip_timeline_read(buf.ctypes.data, buf.nbytes) == 0
        t = buf.reshape(WGS, SLOTS).astype(np.int64)
        decode = t[:, 0] != 0
        t0 = t[decode, 0].min()
        rel = (t - t0) * 0.01
        end = rel[decode, 19].max()
        ends.append(rel[:, 18].copy())
        print(f"call {rep}: {int(decode.sum())} workgroups, span {end:.2f} us", flush=True)
        for k, name in NAMES.items():
            rows = decode
            col = t[rows, k]
            have = col != 0
            if not have.any():
                continue
            r = rel[rows, k][have]
            print(f"  {name:13s} n {int(have.sum()):4d}  min {r.min():7.2f}  med {np.median(r):7.2f}  "
                  f"max {r.max():7.2f}", flush=True)
        # where the late workgroups are: by XCD (workgroup id mod 8)
        ids = np.flatnonzero(decode)
        le = rel[ids, 18]
        per_xcd = " ".join(f"{np.median(le[ids % 8 == x]):.2f}" for x in range(8))
        print(f"  loop end median by XCD: {per_xcd}", flush=True)
    if len(ends) > 1:
        # is a workgroup's lateness a property of its position (same in every
        # call) or of the call?  rank correlation of loop-end times across calls
        live = np.flatnonzero(t[:, 0] != 0)
        a, b = ends[0][live], ends[-1][live]
        ra, rb = a.argsort().argsort(), b.argsort().argsort()
        rho = float(np.corrcoef(ra, rb)[0, 1])
        print(f"loop-end rank correlation between the first and last call: {rho:.3f}", flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--workload", default="int4_gqa_128k")
    ap.add_argument("--calls", type=int, default=3)
    ap.add_argument("--child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.child:
        return child(args)
    if not LIB.exists():
        print(f"{LIB.name} is missing: run python kvssd-attention_amd/csrc/build.py --timeline", file=sys.stderr)
        return 2
    env = dict(os.environ, KVSSD_HIP_LIBRARY=str(LIB))
    cmd = [sys.executable, str(Path(__file__).resolve()), "--child", "--workload", args.workload,
           "--calls", str(args.calls)]
    return subprocess.run(cmd, env=env).returncode


if __name__ == "__main__":
    sys.exit(main())
