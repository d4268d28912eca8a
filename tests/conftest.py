"""Test setup: import paths and the `gpu` marker.

`-m "not gpu"` runs on any machine (oracle pinning, host logic, C-ABI loading);
`-m gpu` runs the HIP parity tests on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (os.path.join(ROOT, "gs-voxelizer_amd"), ROOT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); parity against the oracle")


@pytest.fixture(scope="session")
def device():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device visible")
    return torch.device("cuda:0")


@pytest.fixture(params=["auto", "lsd", "bucket"])
def binning_path(request, monkeypatch):
    """Binning through each of the library's two sort paths (GSV_BINNING: the
    LSD passes, or the split of the boxes' rows into buckets plus per-bucket
    sorts) and through its own choice; both must give the same bits."""
    if request.param == "auto":
        monkeypatch.delenv("GSV_BINNING", raising=False)
    else:
        monkeypatch.setenv("GSV_BINNING", request.param)
    return request.param


@pytest.fixture
def set_chains():
    """A setter of the backward's chained rows for one test
    (gs_voxelizer.cuda.set_backward_chains); the setting before the test is
    restored afterwards."""
    import gs_voxelizer.cuda as _C
    saved = []

    def _set(enabled: bool) -> None:
        prev = _C.set_backward_chains(enabled)
        if not saved:
            saved.append(prev)

    yield _set
    if saved:
        _C.set_backward_chains(saved[0])
