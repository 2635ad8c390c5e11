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
        "int4_gqa_16k", "int4_gqa_32k", "int4_gqa_64k", "int4_gqa_512k", "int4_gqa_2m", "int4_gqa_1m_host_staged",
    ):
        assert name in proc.stdout
    text = " ".join(proc.stdout.split())
    assert "(default 20)" in text
    assert "--settle-ms" in text and "(clock settle; 0 = none)" in text


def test_cpu_baseline_checks_the_timed_step_on_cpu_tensors():
    """cpu_baseline's checks run on the host, against the oracle: fed the torch
    reference backend's result as the timed step it reports ok; a perturbed
    one, an all-zero output and one 10 % short (both within max-abs 2e-3 at
    this output's size) are not ok."""
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
    assert good["kind"] == "port" and good["cores"] >= 1
    assert good["gpu_check"]["ok"] and good["timed_step_check"]["ok"] is True
    assert good["timed_step_check"]["max_abs_out"] < 1e-5 and good["torch_reference"]["ms_per_full_step"] > 0
    bad = bench.cpu_baseline(torch, query, cache, valid, 4, None, budget_s=1.0, timed=(out + 0.1, lse))
    assert bad["timed_step_check"]["ok"] is False and "gpu_check" not in bad
    # outputs far below 2e-3 in magnitude: only the norm-relative check sees these
    small = out * 1e-3
    ref = bench.parity(small.numpy(), lse.numpy(), small.numpy(), lse.numpy())
    assert ref["ok"]
    assert not bench.parity(torch.zeros_like(small).numpy(), lse.numpy(), small.numpy(), lse.numpy())["ok"]
    assert not bench.parity((0.9 * small).numpy(), lse.numpy(), small.numpy(), lse.numpy())["ok"]
    # an lse shifted by 0.105 (a tenth of the tokens dropped) passes rtol 1e-2 at lse ~ 12, not max-abs 2e-3
    assert not bench.parity(out.numpy(), (lse + 0.105).numpy(), out.numpy(), lse.numpy())["ok"]
