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
