"""Test configuration.

``-m "not gpu"`` runs the oracle pinning, host logic, the C-ABI surface and
the native CPU path; ``-m gpu`` runs the HIP parity tests on an MI355X.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
for p in (ROOT, ROOT / "mlx-sparse_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

import torch  # noqa: E402,F401 - HIP runtime first, then the native library


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device)")


def _gpu_present() -> bool:
    try:
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if _gpu_present():
        return
    skip = pytest.mark.skip(reason="no HIP device")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.lib()
    return o


@pytest.fixture(scope="session")
def ms():
    import mlx_sparse

    return mlx_sparse


@pytest.fixture
def cpu(ms):
    """Run mlx_sparse on the CPU device for the duration of a test."""
    prev = ms.default_torch_device()
    ms.use_cpu()
    yield ms
    if prev.type == "cuda":
        ms.use_gpu(prev.index or 0)
    else:
        ms.use_cpu()


@pytest.fixture
def gpu(ms):
    prev = ms.default_torch_device()
    ms.use_gpu()
    yield ms
    if prev.type == "cpu":
        ms.use_cpu()
