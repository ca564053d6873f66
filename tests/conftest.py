import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def gpu():
    """The gfx950 device; GPU tests fail (not skip) when run with -m gpu on a box without it."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU in this process")
    props = torch.cuda.get_device_properties(0)
    arch = getattr(props, "gcnArchName", "")
    assert arch.startswith("gfx950"), f"expected a gfx950 device, found {arch!r}"
    from instinctflash_amd import _lib
    _lib.load()  # raises if the HIP library is not built: no silent fallback
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def oracle_mod():
    import oracle
    oracle.load()
    return oracle


def pytest_report_header(config):
    return f"ifx tests, cwd={os.getcwd()}"
