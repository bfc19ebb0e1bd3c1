"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (run with `-m gpu` on the GPU box); every
other test runs on the CPU. GPU tests call the kernels through the C ABI
(libnspeech_rocm.so via nspeech_amd.abi) and check them against the CPU oracle
(oracle/), the float64 closed forms and the committed fixtures in
tests/golden/.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def dev():
    """The GPU: fails loudly (no CPU fallback) when it or the library is absent."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a GPU")
    from nspeech_amd import abi

    abi.init()
    return torch.device("cuda:0")
