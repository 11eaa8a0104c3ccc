import os
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
for p in (REPO / "mlperf-training_amd", REPO):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:  # pragma: no cover
        return False


@pytest.fixture(scope="session")
def hip_lib():
    """The native library; a GPU test must run on it, never on a fallback."""
    import hstu_amd

    lib = hstu_amd.load_library()
    return lib


@pytest.fixture
def fp8_bwd(monkeypatch):
    """Set the FP8 backward arm's process default for one test, restored after:
    fp8_bwd(enabled=True, uvqk=True, ...) takes Fp8BackwardConfig fields."""
    import hstu_amd.bwd_fp8 as B

    saved = B._default

    def use(**fields):
        cfg = B.Fp8BackwardConfig(**fields)
        B.set_default_config(cfg)
        return cfg

    yield use
    B.set_default_config(saved)
    B.reset_sites()
