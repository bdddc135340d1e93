"""Test configuration: import paths and the `gpu` marker.

Tests marked `gpu` need an MI355X (ROCm torch with a visible device); the
rest run on the CPU.  GPU tests fail, rather than skip, when no GPU is
visible, so a run on a GPU box cannot pass on a silent fallback.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (str(ROOT / "llm-compileforge_amd"), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU (ROCm)")
    config.addinivalue_line("markers", "slow: long-running CPU test")


@pytest.fixture(scope="session")
def gpu():
    import torch

    assert torch.cuda.is_available() and torch.version.hip is not None, "GPU test run without a ROCm GPU"
    dev = torch.device("cuda:0")
    print(f"\n[gpu] {torch.cuda.get_device_name(dev)}", flush=True)
    return dev
