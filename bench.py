"""Decode-step benchmark of the fused INT2/INT4 HIP path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload int4_gqa_128k]

A step is one fused decode (split kernel + merge kernel) of one query token
over the workload's packed KV cache, which is resident in HBM before timing
starts.  Inputs are synthetic and seeded: K/V randn fp16 quantised with the
package's own quantiser on the GPU, query randn fp16.  Several distinct copies
of the packed cache (> 512 MB in total) are rotated across steps so the 256 MB
Infinity Cache cannot serve repeats.

Output: one JSON line.  ``value`` is packed-KV GB/s over the whole step
(algorithmic bytes / step time, the K steps timed back to back with events
only at the two ends, after W untimed warm-up steps).  Before the warm-up the
bench runs untimed back-to-back steps for ``--settle-ms`` (50 ms by default,
reported in ``settle``): an idle GPU needs tens of milliseconds of load to
reach the clocks a continuous decode runs at, and a timed region that starts
inside that ramp reads ~5-8% slow.  ``roofline.achieved`` is the same bytes over the
dominant (split) kernel's average duration: a second pass launches the split
kernel alone K times back to back between two HIP events on its stream.
``step_us`` gives p10 / p50 / p90 of single steps (an event pair around each).
``roofline.attainable`` is the same session's plain streaming-read rate (the
library's read probe over 1 GiB).  ``pipeline`` times the public Python path,
``KVSSDPipeline.decode`` on layers resident in HBM (selection, argument checks
and allocation included; the merge writes the fp16 output itself), over a
store of the workload's shape written to a temporary directory.
``cpu_baseline`` is the reference's CPU decode restated by the oracle (C,
float64 accumulation, OpenMP on every host core: ``kind`` "port") over the
same blocks, with the HIP result and the last timed step's output checked
against it (``gpu_check``, ``timed_step_check``: the contract tolerance, lse
max-abs 2e-3, out norm-relative 1e-2); the portable ``reference`` backend
(torch on CPU tensors) is timed beside it (``torch_reference``).  The default
line (INT4 GQA 128K) also carries ``workloads``: the 4K, INT2 128K and sparse
256K GQA-8 decodes and the host-staged 1M stream, each with its step time,
roofline fraction (PCIe rate for the stream), the oracle's CPU time and a
check of its output against the oracle.

``--workload int4_gqa_1m_host_staged`` times the other regime: 1,048,576
tokens whose raw records sit in page-locked host memory and stream to the GPU
in 64-record chunks (one H2D copy each, alternating between two transfer
streams), each chunk gathered, CRC-checked, decoded and merged on a compute
stream.  Its line reports the step time, the PCIe rate, and copy-only /
compute-only legs from which the overlap follows; it is PCIe-bound, not an
HBM figure.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT / "kvssd-attention_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "µs/decode step + packed-KV HBM GB/s (% peak), INT4 GQA 128K tokens"
# the same measurement on the other decode workloads
WORKLOAD_LABELS = {
    "int4_gqa_128k": "INT4 GQA 128K tokens",
    "int2_gqa_128k": "INT2 GQA 128K tokens",
    "int4_gqa_4k": "INT4 GQA 4K tokens",
    "int4_gqa8_256k_sparse": "INT4 GQA 8, 256K tokens, RecentSinkBlocks(1, 32)",
    "int4_gqa_16k": "INT4 GQA 16K tokens",
    "int4_gqa_32k": "INT4 GQA 32K tokens",
    "int4_gqa_64k": "INT4 GQA 64K tokens",
    "int4_gqa_256k": "INT4 GQA 256K tokens",
    "int4_gqa_512k": "INT4 GQA 512K tokens (HBM-resident)",
    "int4_gqa_1m": "INT4 GQA 1M tokens (HBM-resident)",
    "int4_gqa_2m": "INT4 GQA 2M tokens (HBM-resident)",
}
HBM_PEAK_GBPS = 8000.0

# name -> (tokens, bits, query_heads, value_scale, outlier_fraction, selector (sink, recent) or None)
WORKLOADS = {
    "int4_gqa_4k": (4096, 4, 32, 1.0, 0.0, None),
    "int4_gqa_128k": (131072, 4, 32, 0.5, 0.0, None),
    "int2_gqa_128k": (131072, 2, 32, 1.0, 0.05, None),
    "int4_gqa8_256k_sparse": (262144, 4, 64, 1.0, 0.0, (1, 32)),
    # other context lengths of the same shape, resident in HBM (context-length scaling)
    "int4_gqa_16k": (16384, 4, 32, 0.5, 0.0, None),
    "int4_gqa_32k": (32768, 4, 32, 0.5, 0.0, None),
    "int4_gqa_64k": (65536, 4, 32, 0.5, 0.0, None),
    "int4_gqa_256k": (262144, 4, 32, 0.5, 0.0, None),
    "int4_gqa_512k": (524288, 4, 32, 0.5, 0.0, None),
    "int4_gqa_1m": (1048576, 4, 32, 0.5, 0.0, None),
    "int4_gqa_2m": (2097152, 4, 32, 0.5, 0.0, None),
}
# name -> (tokens, bits, query_heads, stage_blocks): records in page-locked host memory
HOST_STAGED = {
    "int4_gqa_1m_host_staged": (1048576, 4, 32, 64),
}
# name -> (kernel, tokens, bits): the record codec on one layer held in HBM
CODEC = {
    "gather_int4_128k": ("gather", 131072, 4),
    "encode_int4_128k": ("encode", 131072, 4),
    # vLLM block records: 8,388,608 fp16 values (a 64-token block of 32 layers,
    # 8 kv heads, head_dim 128, K and V) as one KVVLLM02 record
    "vllm_encode_int4_8m": ("vllm_encode", 8388608, 4),
    "vllm_decode_int4_8m": ("vllm_decode", 8388608, 4),
}
KV_HEADS, HEAD_DIM, BLOCK_TOKENS, GROUP = 8, 128, 128, 32


def alg_bytes(n_blocks: int, bits: int) -> int:
    """Packed K+V codes plus K+V fp16 scales read per step."""
    per_token_head = 2 * HEAD_DIM * bits // 8 + 2 * (HEAD_DIM // GROUP) * 2
    return n_blocks * BLOCK_TOKENS * KV_HEADS * per_token_head


def make_cache(torch, dev, tokens, bits, qh, value_scale, outliers, seed=7):
    from kvssd.quant import quantize_tensor

    gen = torch.Generator(device=dev).manual_seed(seed)
    out = {}
    for name in ("k", "v"):
        x = torch.randn(tokens, KV_HEADS, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
        x = x * value_scale
        if outliers:
            mask = torch.rand(x.shape, generator=gen, device=dev) < outliers
            x = torch.where(mask, x * 8, x)
        q = quantize_tensor(x, bits, GROUP)
        nb = tokens // BLOCK_TOKENS
        out["p" + name] = q.packed.reshape(nb, BLOCK_TOKENS, KV_HEADS, HEAD_DIM * bits // 8)
        out["s" + name] = q.scales.reshape(nb, BLOCK_TOKENS, KV_HEADS, HEAD_DIM // GROUP)
        del x
    query = torch.randn(qh, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    valid = torch.full((tokens // BLOCK_TOKENS,), BLOCK_TOKENS, dtype=torch.int32, device=dev)
    return query, out, valid


def step_percentiles(torch, stream, step, steps: int) -> dict:
    """p10 / p50 / p90 of single decode steps: an event pair around each of K steps."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for i, (a, b) in enumerate(evs):
        a.record(stream)
        step(i)
        b.record(stream)
    torch.cuda.synchronize()
    us = sorted(a.elapsed_time(b) * 1e3 for a, b in evs)

    def pick(f: float) -> float:
        return round(us[min(len(us) - 1, int(f * len(us)))], 2)

    return {"p10": pick(0.1), "p50": pick(0.5), "p90": pick(0.9), "timing": "an event pair around each of K steps"}


def pipeline_leg(torch, dev, tokens: int, bits: int, qh: int, sel, steps: int, warmup: int, layers: int = 4) -> dict:
    """KVSSDPipeline.decode(query, layer, selector) on layers resident in HBM.

    The public Python path, host work included (selection, argument checks,
    output allocation; the merge stores the fp16 output): a KVCacheStore of ``layers`` layers of
    the workload's shape is written to a temporary directory, every layer is
    made resident, and the steps cycle through the layers as a decode over a
    model's layers does (at 128K tokens the 4 layers, 604 MB, are larger than
    the Infinity Cache; at 4K they fit in it)."""
    import tempfile

    from kvssd import KVCacheStore, KVSSDPipeline
    from kvssd.format import CacheSpec
    from kvssd.selectors import AllBlocks, RecentSinkBlocks

    gen = torch.Generator(device=dev).manual_seed(11)
    spec = CacheSpec(layers, KV_HEADS, HEAD_DIM, BLOCK_TOKENS, bits, GROUP)
    selector = AllBlocks() if sel is None else RecentSinkBlocks(*sel)
    with tempfile.TemporaryDirectory(prefix="kvssd_bench_") as root:
        shape = (layers, tokens, KV_HEADS, HEAD_DIM)
        keys = torch.randn(shape, generator=gen, device=dev, dtype=torch.float16)
        values = torch.randn(shape, generator=gen, device=dev, dtype=torch.float16)
        store = KVCacheStore.create(root, keys, values, spec)
        del keys, values
        query = torch.randn(qh, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
        with store, KVSSDPipeline(store, device=dev, attention_backend="hip") as pipe:
            pipe.load_resident()
            for i in range(warmup):
                pipe.decode(query, i % layers, selector)
            torch.cuda.synchronize()
            # host cost of a call alone: K calls with nothing waited for
            t0 = time.perf_counter()
            for i in range(steps):
                pipe.decode(query, i % layers, selector)
            enqueue = (time.perf_counter() - t0) / steps
            stream = torch.cuda.current_stream(dev)
            start = torch.cuda.Event(enable_timing=True)
            end = torch.cuda.Event(enable_timing=True)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            start.record(stream)
            for i in range(steps):
                out = pipe.decode(query, i % layers, selector)
            end.record(stream)
            torch.cuda.synchronize()
            wall = time.perf_counter() - t0
            kernel = pipe.attention_backend.last_kernel
            ok = bool(torch.isfinite(out).all().item())
    return {
        "us_per_step": round(wall / steps * 1e6, 2),
        "gpu_us_per_step": round(start.elapsed_time(end) * 1e3 / steps, 2),
        "host_enqueue_us_per_call": round(enqueue * 1e6, 2),
        "path": f"KVSSDPipeline.decode over {layers} HBM-resident layers in turn, "
        f"{'AllBlocks' if sel is None else f'RecentSinkBlocks{tuple(sel)}'}, hip backend, fp16 output",
        "kernel": kernel,
        "finite": ok,
    }


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or "unknown"


def parity(out, lse, ref_out, ref_lse) -> dict:
    """The checks every full-size parity test applies: the contract tolerance
    (max-abs 2e-3, rel 1e-2), lse at max-abs 2e-3 with no relative term, and
    out at norm-relative error 1e-2 (which an all-zero or partial output
    cannot pass)."""
    import numpy as np

    out, lse = np.asarray(out, np.float64), np.asarray(lse, np.float64)
    ref_out, ref_lse = np.asarray(ref_out, np.float64), np.asarray(ref_lse, np.float64)
    excess = float(np.max(np.abs(out - ref_out) - 1e-2 * np.abs(ref_out)))
    lse_excess = float(np.max(np.abs(lse - ref_lse) - 1e-2 * np.abs(ref_lse)))
    lse_abs = float(np.max(np.abs(lse - ref_lse)))
    norm_rel = float(np.linalg.norm(out - ref_out) / max(float(np.linalg.norm(ref_out)), 1e-30))
    return {
        "max_abs_out": float(np.max(np.abs(out - ref_out))),
        "max_abs_lse": lse_abs,
        "norm_rel_out": norm_rel,
        "tolerance": "atol 2e-3 + rtol 1e-2 (out, lse); lse max-abs 2e-3; out norm-relative 1e-2",
        "ok": bool(excess <= 2e-3 and lse_excess <= 2e-3 and lse_abs <= 2e-3 and norm_rel <= 1e-2
                   and np.isfinite(out).all()),
    }


def oracle_time(q, arr, valid, bits, sample, threads: int, runs: int = 3):
    """The C oracle (float64 accumulation, OpenMP) over the blocks ``sample``:
    median seconds of ``runs`` timed calls after one warm-up, and its result."""
    import numpy as np

    from oracle import oracle as O

    sel = np.asarray(sample, np.int32)
    scale = 1 / math.sqrt(HEAD_DIM)

    def call():
        return O.attention(q, arr["pk"], arr["pv"], arr["sk"], arr["sv"], valid, bits, GROUP, scale,
                           block_table=sel, threads=threads)

    call()
    times, res = [], None
    for _ in range(runs):
        t0 = time.perf_counter()
        res = call()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], res


def cpu_baseline(torch, query, cache, valid, bits, table, budget_s: float = 4.0, gpu_run=None, timed=None):
    """The CPU baseline: the oracle's C restatement of the reference decode
    (ReferenceAttentionBackend.run: dequantise, scores, softmax, P V; float64
    accumulation, OpenMP over every host core) timed over the workload's
    blocks, 1 warm-up and 3 timed runs, the median reported (``kind`` "port").
    ``gpu_run(ids)`` gives the HIP result over the same blocks, checked here
    against the oracle's; when the sample is the whole step, ``timed`` (the
    last timed step's out and lse) is checked too.  Beside it, the portable
    ``reference`` backend (the reference's torch code path restated, on torch's
    CPU threads) over a sample sized to ~``budget_s`` per run."""
    from kvssd.backends import PackedBatch
    from kvssd.backends.reference import ReferenceAttentionBackend

    cores = os.cpu_count() or 1
    torch.set_num_threads(cores)
    threads = torch.get_num_threads()
    host = {k: t.cpu() for k, t in cache.items()}
    va = valid.cpu()
    q = query.cpu()
    ids = list(range(host["pk"].shape[0])) if table is None else list(table)
    scale = 1 / math.sqrt(HEAD_DIM)
    c_threads = min(cores, 64)
    arr = {k: v.numpy() for k, v in host.items()}
    # the oracle over the whole step when it takes at most ~budget_s, else a
    # prefix of the blocks (extrapolated)
    probe = ids[: min(32, len(ids))]
    t_probe, _ = oracle_time(q.float().numpy(), arr, va.numpy(), bits, probe, c_threads, runs=1)
    n = int(max(1, min(len(ids), budget_s / max(t_probe / len(probe), 1e-9))))
    sample = ids[:n]
    tc, (ref_out, ref_lse) = oracle_time(q.float().numpy(), arr, va.numpy(), bits, sample, c_threads)
    nbytes = alg_bytes(len(sample), bits)
    result = {
        "value": round(nbytes / tc / 1e9, 4),
        "unit": "GB/s",
        "cores": c_threads,
        "kind": "port",
        "sample": f"{len(sample)} of {len(ids)} blocks of the same packed batch through the oracle's C "
        f"restatement of ReferenceAttentionBackend.run (float64 accumulation, OpenMP, {c_threads} threads), "
        f"median of 3 runs after 1 warm-up: {tc * 1e3:.1f} ms each, a full step extrapolates to "
        f"{tc * len(ids) / len(sample) * 1e3:.1f} ms",
        "ms_per_full_step": round(tc * len(ids) / len(sample) * 1e3, 3),
        "os_cpu_count": cores,
        "cpu_model": cpu_model(),
    }
    if gpu_run is not None:
        g_out, g_lse = gpu_run(sample)
        result["gpu_check"] = {**parity(g_out.cpu().numpy(), g_lse.cpu().numpy(), ref_out, ref_lse),
                               "blocks": len(sample)}
    if timed is not None:
        if len(sample) == len(ids):
            t_out, t_lse = (x.cpu().numpy() for x in timed)
            result["timed_step_check"] = parity(t_out, t_lse, ref_out, ref_lse)
        else:
            result["timed_step_check"] = {"ok": None, "why": "the CPU sample is smaller than a step"}

    # the portable reference backend (torch on CPU tensors) over a sample
    # sized from a 16-block probe (its first call pays torch's one-time costs,
    # so it is timed on its second call)
    backend = ReferenceAttentionBackend()

    def run(blocks):
        idx = torch.tensor(blocks, dtype=torch.long)
        batch = PackedBatch(*(host[k].index_select(0, idx) for k in ("pk", "pv", "sk", "sv")), va[idx], bits, GROUP)
        t0 = time.perf_counter()
        out, lse = backend.run(q, batch, scale)
        return time.perf_counter() - t0, out, lse

    probe = ids[: min(16, len(ids))]
    run(probe)
    per_block = run(probe)[0] / len(probe)
    m = int(max(1, min(len(ids), budget_s / max(per_block, 1e-9))))
    tsample = ids[:m]
    run(tsample)  # warm-up
    tt = sorted(run(tsample)[0] for _ in range(3))[1]
    result["torch_reference"] = {
        "value": round(alg_bytes(m, bits) / tt / 1e9, 4),
        "unit": "GB/s",
        "threads": threads,
        "sample": f"{m} of {len(ids)} blocks, kvssd.backends.reference on CPU tensors, median of 3 runs",
        "ms_per_full_step": round(tt * len(ids) / m * 1e3, 3),
    }
    return result


def copy_calibration(torch, dev, nbytes: int, steps: int, warmup: int) -> int:
    """Plain device-to-device copy of a known size: its FETCH_SIZE / WRITE_SIZE
    per dispatch, against nbytes, gives the counters' scale on this GPU."""
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        dst.copy_(src)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    print(json.dumps({"copy_bytes": nbytes, "steps": steps, "ms_per_copy": round(ms, 5),
                      "read_GBps": round(nbytes / ms / 1e6, 1)}), flush=True)
    return 0


def launch_floor(torch, dev, steps: int, warmup: int) -> int:
    """Back-to-back launches of the library's smallest kernel (the code unpack of
    64 packed bytes, one 256-thread workgroup) on one stream between two events:
    the per-launch cost every kernel of a decode step pays on this GPU and
    runtime, whatever its work.  Issued from Python the loop can be host-bound
    (``host_us_per_launch`` says so), so the same launches are also captured in
    a graph and replayed."""
    from kvssd import _native

    lib = _native.load()
    packed = torch.randint(0, 255, (64,), dtype=torch.uint8, device=dev)
    codes = torch.empty(64 * 2, dtype=torch.uint8, device=dev)

    def launch(stream) -> None:
        _native.check(
            lib.kvssd_hip_unpack_codes(packed.data_ptr(), 4, 64, codes.data_ptr(), _native.stream_handle(stream)),
            "unpack_codes",
        )

    stream = torch.cuda.Stream(dev)
    with torch.cuda.stream(stream):
        for _ in range(warmup):
            launch(stream)
    torch.cuda.synchronize()
    n = max(steps, 1000)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        t0 = time.perf_counter()
        start.record(stream)
        for _ in range(n):
            launch(stream)
        end.record(stream)
        host = time.perf_counter() - t0
    torch.cuda.synchronize()
    loop_us = start.elapsed_time(end) * 1e3 / n
    per_graph = 100
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(per_graph):
            launch(stream)
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, n // per_graph)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            graph.replay()
        end.record(stream)
    torch.cuda.synchronize()
    graph_us = start.elapsed_time(end) * 1e3 / (reps * per_graph)
    print(json.dumps({"launch_floor_us": round(loop_us, 3), "host_us_per_launch": round(host * 1e6 / n, 3),
                      "graph_node_us": round(graph_us, 3), "launches": n,
                      "kernel": "unpack_codes_kernel, 64 bytes, one 256-thread workgroup"}), flush=True)
    return 0


def codec(torch, dev, args) -> int:
    """One launch of the record gather (records -> PackedBatch arrays with the
    CRC check) or of the record encoder (fp16 K/V -> records) over one layer
    in HBM; several copies rotate so the Infinity Cache cannot serve repeats."""
    from kvssd.format import CacheSpec
    from kvssd.records_hip import encode_records, gather_records

    kind, tokens, bits = CODEC[args.workload]
    if kind.startswith("vllm"):
        return vllm_codec(torch, dev, args, kind, tokens, bits)
    spec = CacheSpec(1, KV_HEADS, HEAD_DIM, BLOCK_TOKENS, bits, GROUP)
    nb = tokens // BLOCK_TOKENS
    gen = torch.Generator(device=dev).manual_seed(7)
    keys = torch.randn(tokens, KV_HEADS, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    values = torch.randn(tokens, KV_HEADS, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    records, crcs = encode_records(keys, values, spec, layer=0)
    payload = spec.payload_bytes
    copies = args.copies or 4
    if kind == "gather":
        raws = [records.view(-1)] + [records.view(-1).clone() for _ in range(copies - 1)]
        outs = [gather_records(r, spec, nb) for r in raws]

        def launch(i):
            r = raws[i % copies]
            gather_records(r, spec, nb, out=outs[i % copies])

        # header + payload read, four arrays + valid + status written
        nbytes = nb * ((52 + payload) + payload + 8)
        name = "gather_chunked_kernel"
    else:
        ins = [(keys, values)] + [(keys.clone(), values.clone()) for _ in range(copies - 1)]

        def launch(i):
            k, v = ins[i % copies]
            encode_records(k, v, spec, 0)  # allocates its outputs; timed with them

        # fp16 K and V read, whole records written
        nbytes = 2 * tokens * KV_HEADS * HEAD_DIM * 2 + nb * spec.record_bytes
        name = "encode_fused_kernel"
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.steps):
        evs[i][0].record(stream)
        launch(i)
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    ms = sorted(a.elapsed_time(b) for a, b in evs)
    med = ms[len(ms) // 2]
    # the gathered arrays / encoded records are checked against each other once
    ok = True
    if kind == "gather":
        pk, pv, sk, sv, valid, status = outs[0]
        ok = int(status.max()) == 0 and int(valid.min()) == BLOCK_TOKENS
    else:
        again, crc2 = encode_records(keys, values, spec, 0)
        ok = bool(torch.equal(again, records)) and bool(torch.equal(crc2, crcs))
    gbps = nbytes / (med * 1e-3) / 1e9
    print(json.dumps({
        "metric": f"record {kind} GB/s (algorithmic bytes), INT4 128K tokens",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8" if kind == "gather" else "f16",
        "data": "synthetic",
        "config": {"workload": args.workload, "tokens": tokens, "bits": bits, "records": nb,
                   "record_bytes": spec.record_bytes, "alg_bytes_per_step": nbytes, "copies_rotated": copies},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None, "kernel": name},
        "ok": ok,
    }), flush=True)
    return 0


def vllm_codec(torch, dev, args, kind, elements, bits) -> int:
    """Encode (fp16 values -> record) or decode (record -> fp16 values, CRC
    checked) of one vLLM block on the GPU; copies rotate past the Infinity Cache."""
    from kvssd import vllm_codec_hip as V

    gen = torch.Generator(device=dev).manual_seed(7)
    copies = args.copies or 8
    vals = [torch.randn(elements, generator=gen, device=dev, dtype=torch.float16) for _ in range(copies)]
    recs = [V.encode_vllm_block(v, bits=bits, group_size=GROUP) for v in vals]
    payload = elements // GROUP * 2 + elements * bits // 8
    outs = [torch.empty_like(v) for v in vals]
    if kind == "vllm_encode":
        def launch(i):
            V.encode_vllm_block(vals[i % copies], bits=bits, group_size=GROUP)

        nbytes = elements * 2 + recs[0].numel()  # values read, record written
        name = "quantize_kernel + vllm_rows_kernel + vllm_combine_kernel"
    else:
        def launch(i):
            V.decode_vllm_block(recs[i % copies], outs[i % copies])

        nbytes = payload + elements * 2  # payload read, values written
        name = "vllm_rows_kernel + vllm_combine_kernel"
    for i in range(args.warmup):
        launch(i)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(args.steps)]
    for i in range(args.steps):
        evs[i][0].record(stream)
        launch(i)  # decode reads its CRC status back, so each step synchronises
        evs[i][1].record(stream)
    torch.cuda.synchronize()
    med = sorted(a.elapsed_time(b) for a, b in evs)[args.steps // 2]
    V.decode_vllm_block(recs[0], outs[0])
    err = float((outs[0].float() - vals[0].float()).abs().max())
    gbps = nbytes / (med * 1e-3) / 1e9
    print(json.dumps({
        "metric": f"vLLM block {kind.split('_')[1]} GB/s (algorithmic bytes), INT4, {elements} fp16 values",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(med, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": args.workload, "elements": elements, "bits": bits, "group_size": GROUP,
                   "record_bytes": recs[0].numel(), "alg_bytes_per_step": nbytes, "copies_rotated": copies},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 2), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None, "kernel": name},
        "max_abs_round_trip": err,
    }), flush=True)
    return 0


def release_host_memory(torch) -> None:
    """Hand torch's cached page-locked blocks back to the HIP runtime now.

    Tensors made with ``pin_memory=True`` return their blocks to torch's
    caching host allocator when they die; ``torch.cuda.empty_cache()`` empties
    only the device cache, so without this the blocks would be freed by the
    host allocator's static destructor at process exit, inside
    ``__cxa_finalize``, after the HIP runtime (and a profiler's tracing
    hooks) may already be shutting down."""
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    torch._C._host_emptyCache()


def host_staged(torch, dev, args) -> int:
    print(json.dumps(host_staged_line(torch, dev, args.workload, args.steps, args.warmup, args.kernel)), flush=True)
    return 0


def host_staged_line(torch, dev, workload: str, steps: int, warmup: int, kernel: str = "auto") -> dict:
    """Records in page-locked host memory streamed through the staging ring."""
    from kvssd import _native
    from kvssd.backends import PackedBatch
    from kvssd.backends.hip import HipAttentionBackend
    from kvssd.format import CacheSpec
    from kvssd.records_hip import encode_records, gather_records
    from kvssd.staging import HostRecords, RecordStager

    tokens, bits, qh, sb = HOST_STAGED[workload]
    spec = CacheSpec(1, KV_HEADS, HEAD_DIM, BLOCK_TOKENS, bits, GROUP)
    rb = spec.record_bytes
    nb = tokens // BLOCK_TOKENS
    gen = torch.Generator(device=dev).manual_seed(7)
    keys = torch.randn(tokens, KV_HEADS, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    values = torch.randn(tokens, KV_HEADS, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    query = torch.randn(qh, HEAD_DIM, generator=gen, device=dev, dtype=torch.float16)
    records, _ = encode_records(keys, values, spec, layer=0)
    del keys, values
    pinned = torch.empty((nb, rb), dtype=torch.uint8, pin_memory=True)
    pinned.copy_(records)
    host = HostRecords(pinned, list(range(nb)))
    backend = HipAttentionBackend(kernel)
    transfers = [torch.cuda.Stream(dev), torch.cuda.Stream(dev)]
    compute = torch.cuda.Stream(dev)
    stager = RecordStager(spec, dev, sb, backend, transfers, compute)
    fill = stager.host_fill(host)
    scale = 1 / math.sqrt(HEAD_DIM)
    ids = list(range(nb))
    chunks = -(-nb // sb)

    def step():
        return stager.run(query, scale, 0, ids, fill)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    walls, enqueue = [], []
    for _ in range(steps):
        t0 = time.perf_counter()
        out, lse = step()
        torch.cuda.synchronize()
        walls.append(time.perf_counter() - t0)
        enqueue.append(stager.last_enqueue_seconds)
    ms_step = 1e3 * sum(walls) / len(walls)

    # copy-only leg: the same H2D copies on the same two transfer streams,
    # nothing else
    lib = _native.load()
    ths = [_native.stream_handle(t) for t in transfers]

    def copies():
        for c in range(chunks):
            n = min(sb, nb - c * sb)
            dst = stager.slots[c % len(stager.slots)].raw.data_ptr()
            rc = lib.kvssd_hip_memcpy_h2d_async(
                ctypes.c_void_p(dst), ctypes.c_void_p(pinned.data_ptr() + c * sb * rb), n * rb, ths[c % len(ths)]
            )
            _native.check(rc, "h2d")

    reps = max(1, min(steps, 10))
    copies()
    torch.cuda.synchronize()
    t_copy = []
    for _ in range(reps):
        t0 = time.perf_counter()
        copies()
        torch.cuda.synchronize()
        t_copy.append(time.perf_counter() - t0)
    ms_copy = 1e3 * sum(t_copy) / len(t_copy)

    # compute-only leg: the same chunk loop with the copies left out; the
    # slots still hold the last step's records, so every gather, CRC check,
    # decode and merge runs on real records
    no_copy = lambda ids, slot: []  # noqa: E731
    t_comp = []
    for _ in range(reps):
        t0 = time.perf_counter()
        stager.run(query, scale, 0, ids, no_copy)
        torch.cuda.synchronize()
        t_comp.append(time.perf_counter() - t0)
    ms_compute = 1e3 * sum(t_comp) / len(t_comp)
    enqueue_compute = stager.last_enqueue_seconds
    slot_arrays = stager.layout.views(stager.slots[0].batch, spec, sb)
    # the streamed result against one fused call over the whole layer in HBM
    pk, pv, sk, sv, valid, st = gather_records(records.view(-1), spec, nb)
    ref_out, ref_lse = backend.run(query, PackedBatch(pk, pv, sk, sv, valid, bits, GROUP), scale)
    max_abs = float((out - ref_out).abs().max())
    ok = int(st.max()) == 0 and bool(torch.isfinite(out).all())

    h2d_bytes = nb * rb
    packed_bytes = alg_bytes(nb, bits)
    overlap = (ms_copy + ms_compute - ms_step) / min(ms_copy, ms_compute)
    line = {
        "metric": "µs/decode step + H2D GB/s, INT4 GQA 1M tokens host-staged",
        "value": round(packed_bytes / (ms_step * 1e-3) / 1e9, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_step, 4),
        "us_per_step": round(ms_step * 1e3, 1),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "tokens": tokens,
            "bits": bits,
            "kv_heads": KV_HEADS,
            "query_heads": qh,
            "head_dim": HEAD_DIM,
            "block_tokens": BLOCK_TOKENS,
            "group_size": GROUP,
            "stage_blocks": sb,
            "chunks": chunks,
            "record_bytes": rb,
            "h2d_bytes_per_step": h2d_bytes,
            "packed_bytes_per_step": packed_bytes,
            "kernel": backend.kernel_for(query, PackedBatch(*slot_arrays, bits, GROUP), scale),
        },
        "h2d_GBps_in_step": round(h2d_bytes / (ms_step * 1e-3) / 1e9, 2),
        "copy_only": {"ms": round(ms_copy, 4), "GBps": round(h2d_bytes / (ms_copy * 1e-3) / 1e9, 2)},
        "compute_only": {"ms": round(ms_compute, 4), "host_enqueue_ms": round(enqueue_compute * 1e3, 4)},
        "host_enqueue_ms_in_step": round(1e3 * sum(enqueue) / len(enqueue), 4),
        "overlap_frac": round(overlap, 4),
        "max_abs_vs_resident": max_abs,
        "records_ok": ok,
    }
    # the streamed result against the oracle over the same records, whose
    # time over the whole layer is the CPU figure
    arr = {"pk": pk.cpu().numpy(), "pv": pv.cpu().numpy(), "sk": sk.cpu().numpy(), "sv": sv.cpu().numpy()}
    va = valid.cpu().numpy()
    threads = min(os.cpu_count() or 1, 64)
    qf = query.float().cpu().numpy()
    t_all, (ref_o, ref_l) = oracle_time(qf, arr, va, bits, ids, threads, runs=1)
    line["oracle_check"] = parity(out.cpu().numpy(), lse.cpu().numpy(), ref_o, ref_l)
    line["cpu_baseline"] = {"value": round(packed_bytes / t_all / 1e9, 4), "unit": "GB/s", "cores": threads,
                            "kind": "port", "ms_per_full_step": round(t_all * 1e3, 3),
                            "sample": f"all {nb} blocks through the oracle's C restatement (float64, OpenMP), "
                            "one run after one warm-up; records already in memory (no reads, no CRC)"}
    # release the ring, its streams and the page-locked records while the
    # runtime is fully up, not in interpreter teardown
    del stager, fill, host, pinned, transfers, compute
    release_host_memory(torch)
    return line


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument(
        "--warmup",
        type=int,
        default=None,
        help="untimed warm-up steps before the timed ones (default 20)",
    )
    ap.add_argument("--workload", default="int4_gqa_128k", choices=sorted(WORKLOADS) + sorted(HOST_STAGED) + sorted(CODEC))
    ap.add_argument("--kernel", default="auto", choices=["auto", "general", "mfma", "staged"])
    ap.add_argument("--copies", type=int, default=0, help="distinct KV copies rotated across steps (0 = auto)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument(
        "--settle-ms",
        type=float,
        default=50.0,
        help="wall time of untimed back-to-back decode steps before the warm-up steps (clock settle; 0 = none)",
    )
    ap.add_argument(
        "--no-pipeline", action="store_true", help="skip the KVSSDPipeline.decode leg (decode workloads)"
    )
    ap.add_argument(
        "--no-workloads",
        action="store_true",
        help="skip the compact record of the other workloads on the default (INT4 GQA 128K) line",
    )
    ap.add_argument(
        "--copy-calibration",
        type=int,
        default=0,
        metavar="BYTES",
        help="instead of decoding, time a plain device copy of BYTES bytes per step (the reference "
        "reading for scaling rocprof FETCH_SIZE / WRITE_SIZE to bytes)",
    )
    ap.add_argument(
        "--launch-floor",
        action="store_true",
        help="instead of decoding, time back-to-back launches of the library's smallest kernel",
    )
    args = ap.parse_args()
    if args.warmup is None:
        args.warmup = 20
    if args.gpus != 1:
        print(
            "bench.py measures one GPU only: the library has no multi-GPU path "
            "(the decode would shard by kv head or by token range across GPUs)",
            file=sys.stderr,
        )
        return 2

    import torch

    import __graft_entry__

    __graft_entry__.ensure_built()  # a fresh or stale build: build once; otherwise load what is built

    dev = torch.device("cuda", 0)
    if args.copy_calibration:
        return copy_calibration(torch, dev, args.copy_calibration, args.steps, args.warmup)
    if args.launch_floor:
        return launch_floor(torch, dev, args.steps, args.warmup)
    if args.workload in HOST_STAGED:
        return host_staged(torch, dev, args)
    if args.workload in CODEC:
        return codec(torch, dev, args)
    line, ctx = decode_workload(torch, dev, args.workload, args.steps, args.warmup, args.settle_ms, args.kernel,
                                args.copies)
    line["roofline"].update(attainable_read(torch, dev, args.steps))
    tokens, bits, qh, sel, nb = ctx["tokens"], ctx["bits"], ctx["qh"], ctx["sel"], ctx["nb"]
    if not args.no_pipeline:
        # enough layers to pass the Infinity Cache, at most 4 (1 at 1M tokens)
        layers = max(1, min(4, math.ceil(1.2e9 / alg_bytes(nb, bits))))
        line["pipeline"] = pipeline_leg(torch, dev, tokens, bits, qh, sel, args.steps, args.warmup, layers)
    if not args.no_cpu:
        backend, query, batch, scale = ctx["backend"], ctx["query"], ctx["batch"], ctx["scale"]

        def gpu_run(ids):
            out, lse = backend.run(query, batch, scale, block_table=ids)
            torch.cuda.synchronize()
            return out, lse

        arrays = {k: getattr(batch, n) for k, n in
                  (("pk", "packed_k"), ("pv", "packed_v"), ("sk", "scales_k"), ("sv", "scales_v"))}
        line["cpu_baseline"] = cpu_baseline(torch, query, arrays, batch.valid_tokens, bits, ctx["table"],
                                            gpu_run=gpu_run, timed=ctx["timed"])
    del ctx
    release_host_memory(torch)
    if args.workload == "int4_gqa_128k" and not args.no_workloads:
        line["workloads"] = other_workloads(torch, dev, args)
    print(json.dumps(line), flush=True)
    return 0


def attainable_read(torch, dev, steps: int) -> dict:
    """Same-session attainable HBM read rate: the library's plain streaming-read
    probe over 1 GiB (four times the Infinity Cache), K passes back to back
    between two events, median of three such timings."""
    from kvssd import _native

    lib = _native.load()
    nbytes = 1 << 30
    data = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    sink = torch.empty(8192, dtype=torch.int32, device=dev)
    sh = _native.stream_handle(torch.cuda.current_stream(dev))
    n = max(10, min(steps, 50))

    def once():
        _native.check(lib.kvssd_hip_read_probe(data.data_ptr(), nbytes, sink.data_ptr(), sink.numel(), sh),
                      "read_probe")

    for _ in range(3):
        once()
    times = []
    for _ in range(3):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(n):
            once()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / n)
    ms = sorted(times)[1]
    del data, sink
    return {"attainable": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "attainable_what": "plain streaming read (kvssd_hip_read_probe: 1 GiB, 32 KB contiguous pieces per "
            "workgroup, 16-byte non-temporal loads), "
            "same session"}


def decode_workload(torch, dev, workload: str, steps: int, warmup: int, settle_ms: float, kernel: str = "auto",
                    copies: int = 0):
    """One decode workload, KV resident in HBM: the bench line (step time,
    split-kernel time, roofline, step percentiles) and the context the CPU
    legs reuse."""
    from kvssd import _native
    from kvssd.backends import PackedBatch
    from kvssd.backends.hip import HipAttentionBackend
    from kvssd.selectors import RecentSinkBlocks

    tokens, bits, qh, vscale, outl, sel = WORKLOADS[workload]
    query, cache, valid = make_cache(torch, dev, tokens, bits, qh, vscale, outl)
    nb = tokens // BLOCK_TOKENS
    table = None
    if sel is not None:
        table = RecentSinkBlocks(*sel).select(list(range(nb)))
    n_read = nb if table is None else len(table)
    nbytes = alg_bytes(n_read, bits)
    cache_bytes = sum(t.numel() * t.element_size() for t in cache.values())
    copies = copies or max(1, min(16, math.ceil(1.2e9 / max(cache_bytes, 1))))
    if table is not None:
        copies = copies or 8
    batches = [PackedBatch(cache["pk"], cache["pv"], cache["sk"], cache["sv"], valid, bits, GROUP)]
    for _ in range(copies - 1):
        batches.append(PackedBatch(*(cache[k].clone() for k in ("pk", "pv", "sk", "sv")), valid, bits, GROUP))

    backend = HipAttentionBackend(kernel)
    scale = 1 / math.sqrt(HEAD_DIM)
    lib = _native.load()
    tab = None
    if table is not None:
        tab = torch.tensor(table, dtype=torch.int32, device=dev)
    desc = backend.describe(query, batches[0], scale, 0 if tab is None else tab.numel())
    need = ctypes.c_size_t(0)
    _native.check(lib.kvssd_hip_decode_workspace_bytes(ctypes.byref(desc), ctypes.byref(need)), "workspace")
    kern = ctypes.c_int(0)
    _native.check(lib.kvssd_hip_decode_kernel(ctypes.byref(desc), ctypes.byref(kern)), "kernel")
    kernel_name = _native.KERNEL_NAMES[kern.value]
    work = torch.empty(int(need.value), dtype=torch.uint8, device=dev)
    out = torch.empty(qh, HEAD_DIM, dtype=torch.float32, device=dev)
    lse = torch.empty(qh, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev)
    sh = _native.stream_handle(stream)
    tab_ptr = None if tab is None else tab.data_ptr()

    def partials(i: int):
        b = batches[i % copies]
        return lib.kvssd_hip_decode_partials(
            ctypes.byref(desc), query.data_ptr(), b.packed_k.data_ptr(), b.packed_v.data_ptr(),
            b.scales_k.data_ptr(), b.scales_v.data_ptr(), b.valid_tokens.data_ptr(), tab_ptr,
            work.data_ptr(), work.numel(), sh,
        )

    # one decode through the entry point the backend and the stager call,
    # with every pointer read once (and, where the CPython fast-call module is
    # built, without ctypes' per-argument conversions: the host enqueue must
    # stay well below a 4K step's GPU time)
    arrays = [(b.packed_k.data_ptr(), b.packed_v.data_ptr(), b.scales_k.data_ptr(), b.scales_v.data_ptr(),
               b.valid_tokens.data_ptr()) for b in batches]
    tail = (tab_ptr, out.data_ptr(), lse.data_ptr(), work.data_ptr(), work.numel(), sh)
    qptr = query.data_ptr()
    fast = _native.fused_decode_fast()

    if fast is not None:
        fcall, fentry = fast
        daddr = ctypes.addressof(desc)  # desc lives as long as this function's closures

        def step(i: int):
            rc = fcall(fentry, daddr, qptr, *arrays[i % copies], *tail)
            if rc:
                _native.check(rc, "decode")
    else:
        dref = ctypes.byref(desc)

        def step(i: int):
            rc = lib.kvssd_hip_fused_decode(dref, qptr, *arrays[i % copies], *tail)
            if rc:
                _native.check(rc, "decode")

    # clock settle (disclosed in the line): back-to-back decode steps for
    # settle_ms of wall time before the warm-up steps, so that the timed
    # steps see the clocks a continuous decode runs at, not the power-up ramp
    # of an idle GPU
    settle_steps = 0
    if settle_ms > 0:
        t_end = time.perf_counter() + settle_ms / 1e3
        while time.perf_counter() < t_end:
            for _ in range(64):
                step(settle_steps)
                settle_steps += 1
            torch.cuda.synchronize()
    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    # host enqueue cost alone: K launches with nothing waited for (behind the
    # queue the warm-up left, so the GPU never starves the measurement)
    t0 = time.perf_counter()
    for i in range(steps):
        step(i)
    enqueue_us = (time.perf_counter() - t0) / steps * 1e6
    torch.cuda.synchronize()
    # timed region: K back-to-back decode steps, events only at its two ends
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        step(i)
    end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_per_step = start.elapsed_time(end) / steps
    timed_result = (out.clone(), lse.clone())  # the last timed step's output
    # second pass: the split kernel alone, the same K launches back to back
    # between two events on the launch stream: its average duration (plus the
    # dispatch gap between back-to-back launches, ~0.5 us, which rocprof's
    # per-dispatch durations leave out)
    k_start = torch.cuda.Event(enable_timing=True)
    k_end = torch.cuda.Event(enable_timing=True)
    k_start.record(stream)
    for i in range(steps):
        rc = partials(i)
        if rc:
            _native.check(rc, "decode_partials")
    k_end.record(stream)
    torch.cuda.synchronize()
    kern_avg = k_start.elapsed_time(k_end) / steps

    pct = step_percentiles(torch, stream, step, steps)

    gbps = nbytes / (ms_per_step * 1e-3) / 1e9
    achieved = nbytes / (kern_avg * 1e-3) / 1e9
    # the output is compared with the oracle in the cpu_baseline leg
    ok = bool(torch.isfinite(out).all().item())

    traffic = None
    tfile = ROOT / "profiles" / f"traffic_{workload}_{kernel_name}.json"
    if tfile.exists():
        traffic = json.loads(tfile.read_text()).get("hbm_bytes_per_launch")

    line = {
        "metric": METRIC if workload == "int4_gqa_128k"
        else f"µs/decode step + packed-KV HBM GB/s (% peak), {WORKLOAD_LABELS[workload]}",
        "value": round(gbps, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "us_per_step": round(ms_per_step * 1e3, 2),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if kernel_name in ("mfma", "staged") else "f32",
        "data": "synthetic",
        "config": {
            "workload": workload,
            "tokens": tokens,
            "bits": bits,
            "kv_heads": KV_HEADS,
            "query_heads": qh,
            "head_dim": HEAD_DIM,
            "block_tokens": BLOCK_TOKENS,
            "group_size": GROUP,
            "blocks_read": n_read,
            "selector": "all" if sel is None else f"recent_sink{sel}",
            "kernel": kernel_name,
            "kv_copies_rotated": copies,
            "alg_bytes_per_step": nbytes,
        },
        "kernel_us": {"avg": round(kern_avg * 1e3, 2), "timing": "K split launches back to back between two events"},
        "step_us": pct,
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel": f"decode_{kernel_name}",
        },
        "host_wall_ms_per_step": round(wall / steps * 1e3, 4),
        "host_enqueue_us_per_step": round(enqueue_us, 2),
        "host_call": "kvssd_hip_fused_decode via " + ("the CPython fast-call module" if fast is not None else "ctypes"),
        "settle": {"ms": settle_ms, "steps": settle_steps,
                   "what": "untimed back-to-back decode steps before the W warm-up steps"},
        "finite": ok,
    }
    ctx = {"tokens": tokens, "bits": bits, "qh": qh, "sel": sel, "nb": nb, "table": table, "backend": backend,
           "query": query, "batch": batches[0], "scale": scale, "timed": timed_result}
    return line, ctx


# the other decode workloads (4K, INT2 128K, sparse 256K GQA 8), reported compactly beside the headline one
OTHER_WORKLOADS = ("int4_gqa_4k", "int2_gqa_128k", "int4_gqa8_256k_sparse")


def other_workloads(torch, dev, args) -> dict:
    """A compact record of the other decode workloads (4K, INT2 128K, sparse
    256K GQA 8) and the host-staged 1M stream: step and split-kernel times,
    roofline fraction (PCIe rate for the stream), the oracle's CPU time, and
    each timed step's output checked against the oracle."""
    rec = {}
    threads = min(os.cpu_count() or 1, 64)
    # at least 200 timed steps each (a few ms of GPU time), whatever K the
    # main line was asked for: 20 steps of a 23 us decode read ~5 % high
    steps, warmup = max(args.steps, 200), max(args.warmup, 20)
    for w in OTHER_WORKLOADS:
        line, ctx = decode_workload(torch, dev, w, steps, warmup, min(args.settle_ms, 20.0), args.kernel)
        batch, bits = ctx["batch"], ctx["bits"]
        arr = {k: getattr(batch, n).cpu().numpy() for k, n in
               (("pk", "packed_k"), ("pv", "packed_v"), ("sk", "scales_k"), ("sv", "scales_v"))}
        ids = list(range(ctx["nb"])) if ctx["table"] is None else list(ctx["table"])
        t_cpu, (ro, rl) = oracle_time(ctx["query"].float().cpu().numpy(), arr, batch.valid_tokens.cpu().numpy(),
                                      bits, ids, threads)
        t_out, t_lse = (x.cpu().numpy() for x in ctx["timed"])
        rec[w] = {
            "steps": steps,
            "us_per_step": line["us_per_step"],
            "kernel_us": line["kernel_us"]["avg"],
            "roofline_frac": line["roofline"]["frac"],
            "pct_hbm_peak_step": line["pct_hbm_peak"],
            "kernel": line["config"]["kernel"],
            "blocks_read": line["config"]["blocks_read"],
            "cpu_ms": round(t_cpu * 1e3, 3),
            "cpu": f"oracle (C, float64, OpenMP, {threads} threads), whole step, median of 3",
            "timed_step_check": parity(t_out, t_lse, ro, rl),
        }
        del ctx, arr
        release_host_memory(torch)
    hs = "int4_gqa_1m_host_staged"
    # (the first passes over freshly page-locked records run slow: the stream
    # gets the warm-up a standalone run of it has)
    h = host_staged_line(torch, dev, hs, max(5, min(args.steps, 10)), max(8, args.warmup), args.kernel)
    rec[hs] = {
        "us_per_step": h["us_per_step"],
        "h2d_GBps_in_step": h["h2d_GBps_in_step"],
        "copy_only_ms": h["copy_only"]["ms"],
        "compute_only_ms": h["compute_only"]["ms"],
        "overlap_frac": h["overlap_frac"],
        "kernel": h["config"]["kernel"],
        "cpu_ms": h["cpu_baseline"]["ms_per_full_step"],
        "cpu": h["cpu_baseline"]["sample"],
        "oracle_check": h["oracle_check"],
        "records_ok": h["records_ok"],
    }
    return rec


if __name__ == "__main__":
    sys.exit(main())
