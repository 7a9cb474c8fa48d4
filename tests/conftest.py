"""Test setup: the package directory and the repo root (for oracle/) on sys.path, and the `gpu` marker.

Tests marked `gpu` need an MI355X (gfx950) and the built liblowbit_w4.so; they fail (not skip) when either is
missing, so a GPU run can never pass on a silent fallback. Everything else runs on the CPU.
"""
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "lowbit-kernels_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built liblowbit_w4.so")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("a GPU test ran without a visible GPU")
    from lowbit import _native
    _native.lib()                       # raises if the library is not built
    return torch.device("cuda", 0)
