"""bench.py command-line contract (CPU): one GPU only, defaults documented."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def run_bench(*args: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True, text=True, timeout=120)


def test_more_than_one_gpu_exits_with_a_message():
    proc = run_bench("--gpus", "2")
    assert proc.returncode == 2
    assert "one GPU only" in proc.stderr
    assert proc.stdout == ""


def test_help_names_the_workloads_and_the_warmup_and_settle_defaults():
    proc = run_bench("--help")
    assert proc.returncode == 0
    for name in (
        "int4_gqa_128k", "int2_gqa_128k", "int4_gqa_4k", "int4_gqa8_256k_sparse", "int4_gqa_256k", "int4_gqa_1m",
        "int4_gqa_1m_host_staged",
    ):
        assert name in proc.stdout
    text = " ".join(proc.stdout.split())
    assert "(default 20)" in text
    assert "--settle-ms" in text and "(clock settle; 0 = none)" in text


def test_cpu_baseline_checks_the_timed_step_on_cpu_tensors():
    """cpu_baseline's checks run on the host: fed the CPU reference's own result
    as the timed step it reports ok; a perturbed one is not ok."""
    import importlib.util

    import torch

    spec = importlib.util.spec_from_file_location("kvssd_bench", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    from kvssd.backends import PackedBatch
    from kvssd.backends.reference import ReferenceAttentionBackend

    query, cache, valid = bench.make_cache(torch, "cpu", 512, 4, 32, 0.5, 0.0)
    batch = PackedBatch(cache["pk"], cache["pv"], cache["sk"], cache["sv"], valid, 4, bench.GROUP)
    out, lse = ReferenceAttentionBackend().run(query, batch, 1 / 128 ** 0.5)

    def gpu_run(ids):
        return out, lse

    good = bench.cpu_baseline(torch, query, cache, valid, 4, None, budget_s=1.0, gpu_run=gpu_run, timed=(out, lse))
    assert good["gpu_check"]["ok"] and good["timed_step_check"]["ok"] is True
    assert good["timed_step_check"]["max_abs_out"] == 0.0
    bad = bench.cpu_baseline(torch, query, cache, valid, 4, None, budget_s=1.0, timed=(out + 0.1, lse))
    assert bad["timed_step_check"]["ok"] is False and "gpu_check" not in bad
