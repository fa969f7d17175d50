"""Test configuration: the `gpu` marker, import paths, and shared fixtures.

`-m "not gpu"` runs on any CPU host: the oracle against the reference's pins, the host logic,
and the C ABI's load/export/argument checks (no device calls). `-m gpu` runs the HIP kernels
through the C ABI on a gfx950 device and compares them with the oracle.
"""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "h3-hrx_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and the built libh3attn.so")


@pytest.fixture(scope="session")
def dev():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a HIP device"
    import h3attn

    h3attn.lib()  # the HIP library must be present: no fallback
    return torch.device("cuda:0")
