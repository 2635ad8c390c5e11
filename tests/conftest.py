"""Test configuration: import paths, the ``gpu`` marker, shared helpers."""

from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "kvssd-attention_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm MI355X (gfx950) GPU; run with -m gpu")


def pytest_sessionstart(session: pytest.Session) -> None:
    # a fresh checkout has no built library: build it once (hipcc, gfx950);
    # otherwise the tests load what is built
    import __graft_entry__

    __graft_entry__.ensure_built()


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available() and torch.version.hip is not None


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not gpu_available():
        pytest.fail("GPU test selected but no ROCm GPU is visible")
    return torch.device("cuda", 0)


def pytest_runtest_setup(item: pytest.Item) -> None:
    # print the case name before any GPU work, so a fault still names it
    if "gpu" in item.keywords:
        print(f"\n[gpu-case] {item.nodeid}", flush=True)


os.environ.setdefault("PYTHONHASHSEED", "0")
