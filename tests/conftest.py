"""Test setup: the `gpu` marker, the package (imported as `cob_amd`) and the oracle."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libtaskops.so on cuda:0)")


@pytest.fixture(scope="session")
def lib():
    """libtaskops.so, loaded through its C ABI (fails loudly when it is not built)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from cob_amd import capi
    return capi.load()
