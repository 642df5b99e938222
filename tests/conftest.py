import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def require_gfx950():
    """Skip without a GPU; fail on the wrong architecture (reference: require_sm90)."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    arch = torch.cuda.get_device_properties(0).gcnArchName.split(":")[0]
    if arch != "gfx950":
        pytest.fail(f"DSA kernels require MI355X gfx950, found {arch}")
    from cxldsagr_amd import _native

    if not _native.LIBRARY_PATH.exists():
        pytest.fail("libdsa_gfx950.so is not built; run __graft_entry__.build()")


@pytest.fixture
def gpu():
    require_gfx950()
    import torch

    return torch.device("cuda", 0)
