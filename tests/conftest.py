"""Test setup: the wdl package (wan-dit-lab_amd/) and the oracle on sys.path, the `gpu` marker.

GPU tests are marked `gpu` and run on an MI355X; they fail loudly (not skip) when the library is not built.
CPU tests cover the oracle against the reference's known answers, host-side validation and the ABI surface.
"""

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "wan-dit-lab_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and lib/libwdl.so")
    config.addinivalue_line("markers", "slow: long-running")


@pytest.fixture(scope="session")
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("GPU required")
    from wdl import _lib

    _lib.library()  # raises FileNotFoundError when the library is not built
    return torch.device("cuda:0")
