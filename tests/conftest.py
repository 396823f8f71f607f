"""pytest configuration: the `gpu` marker and shared fixtures.

GPU tests run only where a ROCm device is visible (the MI355X box); there they call the
gfx950 library through its C ABI and check it against the CPU oracle. CPU tests pin the
oracle itself and the host-side logic.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

REPO_ROOT = Path(__file__).resolve().parents[1]
if str(REPO_ROOT) not in sys.path:
    sys.path.insert(0, str(REPO_ROOT))


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built libkg_gfx950.so")


def gpu_available() -> bool:
    try:
        import torch
    except ImportError:  # pragma: no cover
        return False
    return bool(torch.cuda.is_available())


@pytest.fixture(scope="session")
def device():
    if not gpu_available():
        pytest.skip("no ROCm device visible")
    import torch

    from kernelcode_generate_amd import native

    native.load_library()  # raises (fails the test) if the HIP library was not built
    native.set_launch_mode(True, None)
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle

    return oracle
