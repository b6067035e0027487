"""Test configuration: the ``gpu`` marker and import paths.

``bayes_ssm`` lives in ``bayes-ssm_amd/`` (not an importable directory name),
and the CPU oracle in ``oracle/``; both are put on ``sys.path`` here.
"""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for sub in (ROOT / "bayes-ssm_amd", ROOT):
    if str(sub) not in sys.path:
        sys.path.insert(0, str(sub))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def cuda_device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture
def rotated_layout(cuda_device):
    """D4M8 float32 calls take the rotated-layout kernels (those the bf16 and float8 entry points share)."""
    from tests._layouts import layout

    with layout("quad"):
        yield
